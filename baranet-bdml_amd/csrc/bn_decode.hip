// bn_decode.hip -- KV-cache decode attention: one new query token per
// sequence against a contiguous per-sequence cache, split-K over the cache.
//
// The reference has no KV cache: generate() re-runs the whole prefix
// (llama_model.py:135-141) and the new token is the last row of the causal
// softmax with seq_offset = L-1 (op_softmax.cuh:89-99).  This kernel computes
// exactly that row for every query head h against KV head
// g = h / (n_heads/n_kv_heads) (llama_layers.hpp:159-163).
//
// Decode is HBM-bound (each cached K/V byte is used by G query heads and
// nothing else), so the design goal is one coalesced pass over the cache:
//   * one workgroup = (sequence b, KV head g, chunk of CH keys); its 4 waves
//     split the chunk; all G query heads of the group are served by the same
//     loads, so every cached byte is read once;
//   * a wave reads 8 (bf16) or 4 (fp32) whole 128/256-byte key rows per
//     16-byte-per-lane load instruction: LPK lanes own one key, each lane 16
//     bytes of it; the q.k partial dot products are reduced across the LPK
//     lanes with xor shuffles;
//   * every lane group keeps its own running (max, sum, acc) per head, updated
//     once per tile of NT keys, and the groups, waves and chunks are merged
//     with the log-sum-exp rule: in-wave by shuffles, in-workgroup through LDS,
//     across chunks by a small combine kernel over (m, l, acc) partials.
// Scores live in the log2 domain: s = (q.k) * scale*log2(e), p = exp2(s - m).
#include "bn_common.hpp"

namespace bn {
namespace {

constexpr int HD = 64;
constexpr int NT = 4;  // keys per lane group between softmax rescales

template <typename T> struct DecVec;
template <> struct DecVec<bf16_t> {
  static constexpr int VEC = 8;
  __device__ static __forceinline__ void load(const bf16_t *p, float (&v)[8]) {
    const uint4 t = *reinterpret_cast<const uint4 *>(p);
    const uint32_t u[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(u[i] << 16);
      v[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
    }
  }
};
template <> struct DecVec<float> {
  static constexpr int VEC = 4;
  __device__ static __forceinline__ void load(const float *p, float (&v)[4]) {
    const float4 t = *reinterpret_cast<const float4 *>(p);
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
  }
};

struct DecodeParams {
  const void *q, *k, *v;
  const int32_t *lens;
  void *o;
  float *ws;  // partials: [batch*n_heads][n_split][HD + 2]
  int batch, max_len, n_heads, n_kv_heads, n_split, chunk;
  float c;  // scale * log2(e)
};

template <typename T, int G>
__global__ __launch_bounds__(256) void decode_split_kernel(DecodeParams p) {
  constexpr int VEC = DecVec<T>::VEC;
  constexpr int LPK = HD / VEC;  // lanes per key
  constexpr int KPI = 64 / LPK;  // keys per wave per load instruction
  __shared__ float red_m[4][G], red_l[4][G];
  __shared__ float red_o[4][G][HD];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int sub = lane % LPK;  // 16-byte slice of the key row
  const int grp = lane / LPK;  // key slot within the wave
  const int split = blockIdx.x % p.n_split;
  const int bg = blockIdx.x / p.n_split;
  const int b = bg / p.n_kv_heads, g = bg % p.n_kv_heads;

  int len = p.lens[b];
  len = len < 0 ? 0 : (len > p.max_len ? p.max_len : len);
  const int k_begin = split * p.chunk;
  if (k_begin >= len) return;  // the combine kernel ignores chunks past len
  const int k_end = min(k_begin + p.chunk, len);

  const int64_t kv_rs = (int64_t)p.n_kv_heads * HD;
  const T *Kb = (const T *)p.k + ((int64_t)b * p.max_len) * kv_rs + (int64_t)g * HD + sub * VEC;
  const T *Vb = (const T *)p.v + ((int64_t)b * p.max_len) * kv_rs + (int64_t)g * HD + sub * VEC;

  // this lane's slice of the G query vectors, pre-scaled into the log2 domain
  float qv[G][VEC];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const T *qp = (const T *)p.q + ((int64_t)b * p.n_heads + g * G + h) * HD + sub * VEC;
    DecVec<T>::load(qp, qv[h]);
#pragma unroll
    for (int e = 0; e < VEC; ++e) qv[h][e] *= p.c;
  }

  float m[G], l[G], acc[G][VEC];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[h][e] = 0.f;
  }

  // keys of this wave: k_begin + wave*KPI*NT + it*4*KPI*NT ..., slot grp
  const int step = 4 * KPI * NT;
  for (int base = k_begin + wave * KPI * NT; base < k_end; base += step) {
    float s[G][NT];
    float kvv[NT][VEC];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int key = base + t * KPI + grp;
      if (key < k_end) {
        DecVec<T>::load(Kb + (int64_t)key * kv_rs, kvv[t]);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) kvv[t][e] = 0.f;
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int key = base + t * KPI + grp;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) d = fmaf(qv[h][e], kvv[t][e], d);
#pragma unroll
        for (int msk = 1; msk < LPK; msk <<= 1) d += __shfl_xor(d, msk, 64);
        s[h][t] = key < k_end ? d : -INFINITY;
      }
    }
    // values for the same keys (zeros past the end: 0 * garbage must not be NaN)
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int key = base + t * KPI + grp;
      if (key < k_end) {
        DecVec<T>::load(Vb + (int64_t)key * kv_rs, kvv[t]);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) kvv[t][e] = 0.f;
      }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float mx = s[h][0];
#pragma unroll
      for (int t = 1; t < NT; ++t) mx = fmaxf(mx, s[h][t]);
      const float m_new = fmaxf(m[h], mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m[h] - m_use);
      m[h] = m_new;
      float pt[NT], ps = 0.f;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        pt[t] = __builtin_amdgcn_exp2f(s[h][t] - m_use);
        ps += pt[t];
      }
      l[h] = l[h] * alpha + ps;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float a = acc[h][e] * alpha;
#pragma unroll
        for (int t = 0; t < NT; ++t) a = fmaf(pt[t], kvv[t][e], a);
        acc[h][e] = a;
      }
    }
  }

  // merge the KPI lane groups of this wave (lanes differing in bits >= log2(LPK))
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float mw = m[h];
#pragma unroll
    for (int msk = LPK; msk < 64; msk <<= 1) mw = fmaxf(mw, __shfl_xor(mw, msk, 64));
    const float mu = mw == -INFINITY ? 0.f : mw;
    const float f = __builtin_amdgcn_exp2f(m[h] - mu);
    float lw = l[h] * f;
#pragma unroll
    for (int msk = LPK; msk < 64; msk <<= 1) lw += __shfl_xor(lw, msk, 64);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float a = acc[h][e] * f;
#pragma unroll
      for (int msk = LPK; msk < 64; msk <<= 1) a += __shfl_xor(a, msk, 64);
      acc[h][e] = a;
    }
    if (lane == 0) {
      red_m[wave][h] = mw;
      red_l[wave][h] = lw;
    }
    if (grp == 0) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) red_o[wave][h][sub * VEC + e] = acc[h][e];
    }
  }
  __syncthreads();

  // merge the 4 waves and write this chunk's partial (m, l, acc[HD]) per head
  for (int idx = tid; idx < G * HD; idx += 256) {
    const int h = idx / HD, d = idx % HD;
    float M = red_m[0][h];
#pragma unroll
    for (int w2 = 1; w2 < 4; ++w2) M = fmaxf(M, red_m[w2][h]);
    const float Mu = M == -INFINITY ? 0.f : M;
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < 4; ++w2) {
      const float f = __builtin_amdgcn_exp2f(red_m[w2][h] - Mu);
      L += red_l[w2][h] * f;
      A += red_o[w2][h][d] * f;
    }
    float *part = p.ws + (((int64_t)b * p.n_heads + g * G + h) * p.n_split + split) * (HD + 2);
    part[2 + d] = A;
    if (d == 0) {
      part[0] = M;
      part[1] = L;
    }
  }
}

// bf16 cache: matrix-core version.  Per wave, tiles of 32 keys:
//   S^T[key][head] = K[key][:] . Q[head][:]   two v_mfma_f32_16x16x32_bf16 per
//     16 keys; the K tile is the A operand straight from HBM (lane: key l%16,
//     16 bytes of d), the G query heads are the B operand columns (padded to 16);
//   online softmax per head column (4 keys per lane, 4 lane groups);
//   O^T[d][head] += V^T[d][key] . P^T[key][head]  one MFMA per 16 d; V^T comes
//     from a per-wave LDS tile written transposed, P^T straight from registers.
// The next tile's K/V loads are issued before the current tile is computed.
typedef __bf16 dbf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 dbf16x4_t __attribute__((ext_vector_type(4)));
typedef float df32x4_t __attribute__((ext_vector_type(4)));
constexpr int TK = 32;   // keys per wave tile
constexpr int VTP = 36;  // V^T LDS pitch (elements): conflict-free writes and b64 reads

template <int G>
__global__ __launch_bounds__(256) void decode_bf16_mfma_kernel(DecodeParams p) {
  __shared__ __attribute__((aligned(16))) bf16_t Vt[4][HD * VTP];
  __shared__ float red_m[4][G], red_l[4][G];
  __shared__ float red_o[4][G][HD];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, grp = lane >> 4;
  const int split = blockIdx.x % p.n_split;
  const int bg = blockIdx.x / p.n_split;
  const int b = bg / p.n_kv_heads, g = bg % p.n_kv_heads;

  int len = p.lens[b];
  len = len < 0 ? 0 : (len > p.max_len ? p.max_len : len);
  const int k_begin = split * p.chunk;
  if (k_begin >= len) return;  // the combine kernel ignores chunks past len
  const int k_end = min(k_begin + p.chunk, len);
  const int ntiles = (k_end - k_begin + TK - 1) / TK;

  const int64_t kv_rs = (int64_t)p.n_kv_heads * HD;
  const bf16_t *Kb = (const bf16_t *)p.k + (int64_t)b * p.max_len * kv_rs + (int64_t)g * HD + 8 * grp;
  const bf16_t *Vb = (const bf16_t *)p.v + (int64_t)b * p.max_len * kv_rs + (int64_t)g * HD + 8 * grp;

  // B operand of S^T: column l16 = query head g*G + l16 (zero past G), d = 8grp + 32t + 0..7
  dbf16x8_t qb[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    if (l16 < G)
      qb[t] = *(const dbf16x8_t *)((const bf16_t *)p.q +
                                   ((int64_t)b * p.n_heads + g * G + l16) * HD + 8 * grp + 32 * t);
    else
      qb[t] = dbf16x8_t{};
  }

  uint4 kr[2][2], vr[2][2];  // [16-key half u][d half t], this lane: key 16u + l16
  auto gload = [&](int kb) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int key = kb + 16 * u + l16;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (key < k_end) {
          kr[u][t] = *(const uint4 *)(Kb + (int64_t)key * kv_rs + 32 * t);
          vr[u][t] = *(const uint4 *)(Vb + (int64_t)key * kv_rs + 32 * t);
        } else {  // zeros: a masked key must not bring NaN/Inf into P.V
          kr[u][t] = make_uint4(0, 0, 0, 0);
          vr[u][t] = make_uint4(0, 0, 0, 0);
        }
      }
    }
  };

  float m = -INFINITY, l = 0.f;
  df32x4_t o[4] = {df32x4_t{}, df32x4_t{}, df32x4_t{}, df32x4_t{}};
  bf16_t *vt = Vt[wave];
  const float c = p.c;

  if (wave < ntiles) gload(k_begin + TK * wave);
  for (int ti = wave; ti < ntiles; ti += 4) {
    const int kb = k_begin + TK * ti;
    uint4 kc[2][2], vc[2][2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        kc[u][t] = kr[u][t];
        vc[u][t] = vr[u][t];
      }
    if (ti + 4 < ntiles) gload(kb + 4 * TK);

    // V tile -> LDS, transposed: vt[d][key], d = 8grp + 32t + e, key = 16u + l16.
    // The tile is private to this wave; LDS operations of a wave complete in order.
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint32_t w4[4] = {vc[u][t].x, vc[u][t].y, vc[u][t].z, vc[u][t].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vt[(8 * grp + 32 * t + 2 * e) * VTP + 16 * u + l16] = (bf16_t)(w4[e] & 0xffffu);
          vt[(8 * grp + 32 * t + 2 * e + 1) * VTP + 16 * u + l16] = (bf16_t)(w4[e] >> 16);
        }
      }

    // S^T: s[u][i] = key kb + 16u + 4grp + i, head column l16
    df32x4_t s[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      s[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(dbf16x8_t, kc[u][0]),
                                                     qb[0], df32x4_t{}, 0, 0, 0);
      s[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(dbf16x8_t, kc[u][1]),
                                                     qb[1], s[u], 0, 0, 0);
    }
    if (kb + TK > k_end) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (kb + 16 * u + 4 * grp + i >= k_end) s[u][i] = -INFINITY;
    }
    float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                     fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float mc = m_use * c;
    const float alpha = __builtin_amdgcn_exp2f(m * c - mc);
    float rs = 0.f;
    dbf16x8_t pb;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = __builtin_amdgcn_exp2f(fmaf(s[u][i], c, -mc));
        rs += e;
        pb[4 * u + i] = (__bf16)e;  // k-slot (grp, 4u+i) = key 16u + 4grp + i
      }
    l = l * alpha + rs;  // this lane group's keys; groups are summed at the end
    m = m_new;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      o[dt] *= alpha;
      const bf16_t *row = vt + (16 * dt + l16) * VTP + 4 * grp;
      const dbf16x4_t lo = *(const dbf16x4_t *)(row);       // keys 4grp .. +3
      const dbf16x4_t hi = *(const dbf16x4_t *)(row + 16);  // keys 16 + 4grp .. +3
      const dbf16x8_t a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, o[dt], 0, 0, 0);
    }
  }

  // o[dt][i] = O^T[d = 16dt + 4grp + i][head l16]; m is uniform over lane groups
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (l16 < G) {
    if (grp == 0) {
      red_m[wave][l16] = m;
      red_l[wave][l16] = l;
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) red_o[wave][l16][16 * dt + 4 * grp + i] = o[dt][i];
  }
  __syncthreads();
  for (int idx = tid; idx < G * HD; idx += 256) {
    const int h = idx / HD, d = idx % HD;
    float M = red_m[0][h];
#pragma unroll
    for (int w2 = 1; w2 < 4; ++w2) M = fmaxf(M, red_m[w2][h]);
    const float Mu = M == -INFINITY ? 0.f : M;
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < 4; ++w2) {
      const float f = __builtin_amdgcn_exp2f((red_m[w2][h] - Mu) * c);
      L += red_l[w2][h] * f;
      A += red_o[w2][h][d] * f;
    }
    float *part = p.ws + (((int64_t)b * p.n_heads + g * G + h) * p.n_split + split) * (HD + 2);
    part[2 + d] = A;
    if (d == 0) {
      part[0] = M * c;  // partials carry the max in the log2 domain
      part[1] = L;
    }
  }
}

// One thread per (b, head, d): merge the chunks [0, ceil(len/chunk)).
template <typename T>
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeParams p) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)p.batch * p.n_heads * HD) return;
  const int d = (int)(idx % HD);
  const int64_t bh = idx / HD;
  const int b = (int)(bh / p.n_heads);
  int len = p.lens[b];
  len = len < 0 ? 0 : (len > p.max_len ? p.max_len : len);
  const int nvalid = (len + p.chunk - 1) / p.chunk;
  const float *part = p.ws + bh * p.n_split * (HD + 2);
  float M = -INFINITY;
  for (int s = 0; s < nvalid; ++s) M = fmaxf(M, part[s * (HD + 2)]);
  const float Mu = M == -INFINITY ? 0.f : M;
  float L = 0.f, A = 0.f;
  for (int s = 0; s < nvalid; ++s) {
    const float *ps = part + s * (HD + 2);
    const float f = __builtin_amdgcn_exp2f(ps[0] - Mu);
    L += ps[1] * f;
    A += ps[2 + d] * f;
  }
  const float out = L > 0.f ? A / L : 0.f;  // empty sequence -> zeros
  Elem<T>::store((T *)p.o + idx, out);
}

int choose_chunk(int batch, int max_len, int n_kv_heads) {
  // enough workgroups to cover 256 CUs several times, chunks >= 128 keys
  int chunk = 1024;
  while (chunk > 128 &&
         (int64_t)batch * n_kv_heads * ((max_len + chunk - 1) / chunk) < 1024)
    chunk >>= 1;
  return chunk;
}

template <typename T, int G>
void launch_split(const DecodeParams &p, dim3 grid, hipStream_t s) {
  if constexpr (std::is_same<T, bf16_t>::value)
    hipLaunchKernelGGL((decode_bf16_mfma_kernel<G>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((decode_split_kernel<T, G>), grid, dim3(256), 0, s, p);
}

template <typename T>
int launch_decode(const DecodeParams &p, int G, hipStream_t s) {
  const dim3 grid((unsigned)((int64_t)p.batch * p.n_kv_heads * p.n_split));
  switch (G) {
    case 1: launch_split<T, 1>(p, grid, s); break;
    case 2: launch_split<T, 2>(p, grid, s); break;
    case 4: launch_split<T, 4>(p, grid, s); break;
    default: launch_split<T, 8>(p, grid, s); break;
  }
  BN_LAUNCH_CHECK();
  const int64_t n = (int64_t)p.batch * p.n_heads * HD;
  hipLaunchKernelGGL(decode_combine_kernel<T>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     s, p);
  BN_LAUNCH_CHECK();
  return BN_OK;
}

}  // namespace
}  // namespace bn

using namespace bn;

extern "C" {

size_t bn_gqa_decode_workspace_size(int batch, int max_len, int n_heads, int head_dim) {
  if (batch <= 0 || max_len <= 0 || n_heads <= 0 || head_dim != HD) return 0;
  // n_split does not depend on n_kv_heads by more than the chunk choice; size
  // for the smallest chunk (most splits) so any n_kv_heads fits
  const int64_t n_split = (max_len + 127) / 128;
  return (size_t)batch * n_heads * n_split * (HD + 2) * sizeof(float);
}

int bn_gqa_decode(int dtype, const void *q, const void *k_cache, const void *v_cache,
                  const int32_t *seq_lens, void *o, int batch, int max_len, int n_heads,
                  int n_kv_heads, int head_dim, float scale, void *workspace,
                  size_t workspace_bytes, void *stream) {
  const char *op = "GQA decode";
  if (dtype != BN_F32 && dtype != BN_BF16)
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": dtype must be F32 or BF16");
  if (batch < 0 || max_len < 0)
    return fail(BN_ERR_SHAPE, std::string(op) + ": negative batch or cache length");
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0)
    return fail(BN_ERR_SHAPE, std::string(op) + ": num_heads must be a positive multiple of num_kv_heads");
  const int G = n_heads / n_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8)
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": heads per KV head must be 1, 2, 4 or 8");
  if (head_dim != HD) return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": head_dim must be 64");
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(BN_ERR_INVALID_ARG, std::string(op) + ": scale must be positive and finite");
  if (batch == 0) return BN_OK;
  if (max_len == 0) return fail(BN_ERR_SHAPE, std::string(op) + ": max_len must be positive");
  if (!q || !k_cache || !v_cache || !seq_lens || !o)
    return fail(BN_ERR_INVALID_ARG, std::string(op) + ": NULL pointer");
  if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15u)
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": q and caches must be 16-byte aligned");
  DecodeParams p;
  p.q = q; p.k = k_cache; p.v = v_cache; p.lens = seq_lens; p.o = o;
  p.batch = batch; p.max_len = max_len; p.n_heads = n_heads; p.n_kv_heads = n_kv_heads;
  p.chunk = choose_chunk(batch, max_len, n_kv_heads);
  p.n_split = (max_len + p.chunk - 1) / p.chunk;
  p.c = scale * 1.4426950408889634f;
  const size_t need = (size_t)batch * n_heads * p.n_split * (HD + 2) * sizeof(float);
  if (workspace && workspace_bytes < need)
    return fail(BN_ERR_INVALID_ARG, std::string(op) + ": workspace of " +
                                        std::to_string(workspace_bytes) + " bytes, need " +
                                        std::to_string(need));
  int st = ensure_device();
  if (st) return st;
  hipStream_t s = as_stream(stream);
  void *ws = workspace;
  bool own = false;
  if (!ws) {
    if ((st = bn_alloc(&ws, need, stream))) return st;
    own = true;
  }
  p.ws = (float *)ws;
  st = dtype == BN_BF16 ? launch_decode<bf16_t>(p, G, s) : launch_decode<float>(p, G, s);
  if (own) {
    int st2 = bn_free(ws, stream);
    if (st == BN_OK) st = st2;
  }
  return st;
}

}  // extern "C"
