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

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <mutex>
#include <vector>

#include "bn_common.hpp"

// Chunk partials of bn_gqa_decode_noalloc: a file-scope device array, one
// copy per GPU, held until the process ends.  Host code never passes its name
// to a kernel (on the host the name is only a stand-in); it uses the device
// address hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) float scratch[BN_GQA_DECODE_SCRATCH_BYTES / sizeof(float)];

// Per-(sequence, query head) split counters of the short-cache decode's
// in-launch merge: slots of kShortMaxUnits counters, zero at load time, a
// host-side ring of slots; each unit's last split clears its counter.
static __device__ __align__(256) uint32_t short_counters[16 * 256];

// bf16 K/V cache loads are non-temporal (streamed once, kept out of L2/MALL):
// +24% on config 3 against plain loads.

namespace bn {
namespace {

constexpr int HD = 64;
constexpr int NT = 8;  // keys per lane group between softmax rescales
// short-cache split (DEC_SHORT): keys per lane group per round (one round
// covers a 640-key cache's 160-key splits: 4 waves x 4 lane groups x 10),
// waves per workgroup and query heads per workgroup
constexpr int kShortNT = 10, kShortWV = 4, kShortG = 1;

template <typename T> struct DecVec;
template <> struct DecVec<float> {
  static constexpr int VEC = 4;
  __device__ static __forceinline__ void load(const float *p, float (&v)[4]) {
    const float4 t = *reinterpret_cast<const float4 *>(p);
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
  }
};

// Sum over each group of N (8 or 16) consecutive lanes with DPP moves inside
// a 16-lane row (no LDS round trip): quad xor 1, quad xor 2, half-row mirror
// (lane i <-> 7 - i), row mirror (lane i <-> 15 - i); every lane gets the sum.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xf, 0xf, false));
}
template <int N>
__device__ __forceinline__ float row_sum(float x) {
  static_assert(N == 8 || N == 16, "8 or 16 lanes");
  x += dpp_mov<0xB1>(x);   // quad_perm 1,0,3,2
  x += dpp_mov<0x4E>(x);   // quad_perm 2,3,0,1
  x += dpp_mov<0x141>(x);  // row_half_mirror
  if (N == 16) x += dpp_mov<0x140>(x);  // row_mirror
  return x;
}

struct DecodeParams {
  const void *q, *k, *v;
  const int32_t *lens;
  void *o;
  float *ws;  // partials: [batch*n_heads][n_split][HD + 2]
  int batch, max_len, n_heads, n_kv_heads, n_split, chunk;
  float c;        // scale * log2(e)
  int hlen = -1;  // >= 0: every sequence's length, from the host (lens not read)
  // cache strides in elements: sequence, KV head, key row (a contiguous
  // [batch, max_len, n_kv_heads, 64] cache: max_len*n_kv_heads*64, 64,
  // n_kv_heads*64; a head-major [batch, n_kv_heads, max_len, 64] one:
  // n_kv_heads*max_len*64, max_len*64, 64)
  int64_t kv_bs = 0, kv_hs = 0, kv_rs = 0;
  // DEC_SHORT: per-(sequence, query head) counters (zero at launch, cleared
  // again by each unit's last split): the last split to arrive merges the
  // unit's records and writes the output in the same launch; null: the
  // records are left for a combine
  uint32_t *cnt = nullptr;
};

// WV waves per workgroup; MODE:
//   DEC_SPLIT: one workgroup per (sequence, KV head, chunk of p.chunk keys)
//     serving the KV head's G query heads; the waves interleave blocks of
//     KPI*NT keys over the chunk; writes the chunk's partial records.
//   DEC_SHORT: one workgroup per (sequence, G query heads of one KV head,
//     split); split s takes keys [s*chunk, (s+1)*chunk) of the sequence's
//     length with chunk = short_split_chunk(len, n_split), each wave a
//     contiguous part; writes the split's partial records.  For short caches
//     and few sequences, where one workgroup per query head is bound by what
//     one compute unit can stream (every workgroup reads the whole cache).
// The workgroups that read the same cache rows (the query heads of one KV
// head, in SHORT) get consecutive unit numbers, and units are
// numbered so that consecutive ones go to one XCD (workgroups are dealt to
// the 8 XCDs in turn): they read those rows from one L2.
constexpr int DEC_SPLIT = 0, DEC_SHORT = 1;
template <typename T, int G, int WV, int MODE>
__global__ __launch_bounds__(64 * WV) void decode_split_kernel(DecodeParams p) {
  constexpr bool CONTIG = MODE == DEC_SHORT;
  constexpr int VEC = DecVec<T>::VEC;
  constexpr int NT = CONTIG ? kShortNT : bn::NT;
  constexpr int LPK = HD / VEC;  // lanes per key
  constexpr int KPI = 64 / LPK;  // keys per wave per load instruction
  __shared__ float red_m[WV][G], red_l[WV][G];
  __shared__ float red_o[WV][G][HD];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int sub = lane % LPK;  // 16-byte slice of the key row
  const int grp = lane / LPK;  // key slot within the wave
  int u = blockIdx.x;
  if (CONTIG && (gridDim.x & 7) == 0) u = (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
  int b, g, h0, split = 0;
  if constexpr (MODE == DEC_SPLIT) {
    split = u % p.n_split;
    const int bg = u / p.n_split;
    b = bg / p.n_kv_heads;
    g = bg % p.n_kv_heads;
    h0 = g * G;
  } else {  // units (sequence, KV head, split, query-head group), the last fastest
    const int qpg = p.n_heads / p.n_kv_heads / G;  // query-head groups per KV head
    const int qg = u % qpg;
    u /= qpg;
    split = u % p.n_split;
    u /= p.n_split;
    g = u % p.n_kv_heads;
    b = u / p.n_kv_heads;
    h0 = g * (p.n_heads / p.n_kv_heads) + qg * G;
  }

  // this lane's slice of the G query vectors, pre-scaled into the log2
  // domain; requested before the length (its loads do not wait for it)
  float qv[G][VEC];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const T *qp = (const T *)p.q + ((int64_t)b * p.n_heads + h0 + h) * HD + sub * VEC;
    DecVec<T>::load(qp, qv[h]);
  }
  int len = p.hlen >= 0 ? p.hlen : p.lens[b];
  len = len < 0 ? 0 : (len > p.max_len ? p.max_len : len);
  const int chunk = MODE == DEC_SHORT ? short_split_chunk(len, p.n_split) : p.chunk;
  const int k_begin = split * chunk;
  if (k_begin >= len) {  // the combine ignores chunks past len
    if (MODE == DEC_SHORT && p.cnt && len == 0 && split == 0)  // no key, no merge: zeros
      for (int idx = tid; idx < G * HD; idx += 64 * WV)
        Elem<T>::store((T *)p.o + ((int64_t)b * p.n_heads + h0) * HD + idx, 0.f);
    return;
  }
  const int k_end = min(k_begin + chunk, len);
  // CONTIG: wave w takes keys [kw0, kw1), a contiguous range; else the waves
  // interleave blocks of KPI*NT keys over the chunk
  const int per = ((k_end - k_begin + WV - 1) / WV + KPI - 1) / KPI * KPI;
  const int kw0 = CONTIG ? k_begin + wave * per : k_begin + wave * KPI * NT;
  const int kw1 = CONTIG ? min(kw0 + per, k_end) : k_end;

  const int64_t kv_rs = p.kv_rs;
  const T *Kb = (const T *)p.k + b * p.kv_bs + g * p.kv_hs + sub * VEC;
  const T *Vb = (const T *)p.v + b * p.kv_bs + g * p.kv_hs + sub * VEC;

#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < VEC; ++e) qv[h][e] *= p.c;

  float m[G], l[G], acc[G][VEC];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[h][e] = 0.f;
  }

  const int step = CONTIG ? KPI * NT : WV * KPI * NT;
  for (int base = kw0; base < kw1; base += step) {
    // K and V of the NT keys of this lane group are requested together (one
    // memory round trip per NT keys); keys past the chunk read the chunk's
    // last row (initialised data, finite) and are masked to P = 0
    float s[G][NT];
    float kk[NT][VEC], vv[NT][VEC];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int key = min(base + t * KPI + grp, kw1 - 1);
      DecVec<T>::load(Kb + (int64_t)key * kv_rs, kk[t]);
      DecVec<T>::load(Vb + (int64_t)key * kv_rs, vv[t]);
    }
    // contiguous ranges: every load of the round is issued before any is
    // consumed.  Left alone, the scheduler trades them for registers (load,
    // wait, use, next: one round trip per key).
    if constexpr (CONTIG) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int key = base + t * KPI + grp;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) d = fmaf(qv[h][e], kk[t][e], d);
        d = row_sum<LPK>(d);
        s[h][t] = key < kw1 ? d : -INFINITY;
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
        for (int t = 0; t < NT; ++t) a = fmaf(pt[t], vv[t][e], a);
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

  // merge the waves and write this chunk's partial (m, l, acc[HD]) per head
  for (int idx = tid; idx < G * HD; idx += 64 * WV) {
    const int h = idx / HD, d = idx % HD;
    float M = red_m[0][h];
#pragma unroll
    for (int w2 = 1; w2 < WV; ++w2) M = fmaxf(M, red_m[w2][h]);
    const float Mu = M == -INFINITY ? 0.f : M;
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < WV; ++w2) {
      const float f = __builtin_amdgcn_exp2f(red_m[w2][h] - Mu);
      L += red_l[w2][h] * f;
      A += red_o[w2][h][d] * f;
    }
    float *part = p.ws + (((int64_t)b * p.n_heads + h0 + h) * p.n_split + split) * kDecRec;
    if (MODE == DEC_SHORT && p.cnt) {  // through to memory: another workgroup merges them
      __hip_atomic_store(part + 2 + d, A, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      if (d == 0) {
        __hip_atomic_store(part, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(part + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      }
      continue;
    }
    part[2 + d] = A;
    if (d == 0) {
      part[0] = M;
      part[1] = L;
    }
  }
  if constexpr (MODE == DEC_SHORT) {
    if (!p.cnt) return;
    // the unit's splits holding keys count themselves; the last to arrive
    // reads their records past the caches and merges them as the combine
    // kernel does (DecMerge), so the output has the combine's bits
    __shared__ bool s_last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's record stores done
    __syncthreads();
    if (tid == 0) {
      const int unit = (b * p.n_heads + h0) / G;
      const uint32_t nvalid = (uint32_t)((len + chunk - 1) / chunk);
      const uint32_t seen = __hip_atomic_fetch_add(p.cnt + unit, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool last = seen == nvalid - 1;
      if (last) __hip_atomic_store(p.cnt + unit, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = last;
    }
    __syncthreads();
    if (!s_last) return;
    const int nvalid = (len + chunk - 1) / chunk;
    for (int idx = tid; idx < G * HD / 4; idx += 64 * WV) {
      const int h = idx / (HD / 4), d0 = (idx % (HD / 4)) * 4;
      const float *part = p.ws + ((int64_t)b * p.n_heads + h0 + h) * p.n_split * kDecRec;
      DecMerge mg;
      mg.load8<true>(part, p.n_split, 0, d0);
      mg.start();
      mg.merge8(0, nvalid);
      for (int s0 = 8; s0 < nvalid; s0 += 8) {
        mg.load8<true>(part, p.n_split, s0, d0);
        mg.merge8(s0, nvalid);
      }
      const float4 r = mg.result();
      T *out = (T *)p.o + ((int64_t)b * p.n_heads + h0 + h) * HD + d0;
      Elem<T>::store(out + 0, r.x);
      Elem<T>::store(out + 1, r.y);
      Elem<T>::store(out + 2, r.z);
      Elem<T>::store(out + 3, r.w);
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

constexpr int NBUF = 2;  // register tile buffers in turn
// register budget for 3 waves per SIMD
template <int G>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
void decode_bf16_mfma_kernel(DecodeParams p) {
  // per-wave V^T tile; after the wave's last tile the same bytes hold its
  // (acc) merge values, so the workgroup needs no second LDS array
  __shared__ __attribute__((aligned(16))) bf16_t Vt[4][HD * VTP];
  __shared__ float red_m[4][G], red_l[4][G];
  static_assert(G * HD * sizeof(float) <= HD * VTP * sizeof(bf16_t), "merge area");

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

  const int64_t kv_rs = p.kv_rs;
  const bf16_t *Kb = (const bf16_t *)p.k + b * p.kv_bs + g * p.kv_hs + 8 * grp;
  const bf16_t *Vb = (const bf16_t *)p.v + b * p.kv_bs + g * p.kv_hs + 8 * grp;

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

  // NBUF register tile buffers used in turn: while one tile is computed, the
  // loads of the other NBUF-1 (and the refill of this one) are in flight
  uint4 kr[NBUF][2][2], vr[NBUF][2][2];  // [buffer][16-key half u][d half t]; lane: key 16u + l16
  // Branch-free loads: a key past the end reads the last valid key instead
  // (its score is masked to -inf, so P = 0 multiplies finite cache data).  A
  // conditional load would make the compiler wait for every outstanding load
  // at the first use, serialising the two buffers.
  auto gload = [&](int buf, int kb) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int key = min(kb + 16 * u + l16, k_end - 1);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        kr[buf][u][t] = *(const uint4 *)(Kb + (int64_t)key * kv_rs + 32 * t);
        vr[buf][u][t] = *(const uint4 *)(Vb + (int64_t)key * kv_rs + 32 * t);
      }
    }
  };

  float m = -INFINITY, l = 0.f;
  df32x4_t o[4] = {df32x4_t{}, df32x4_t{}, df32x4_t{}, df32x4_t{}};
  bf16_t *vt = Vt[wave];
  const float c = p.c;

  auto compute = [&](int buf, int kb) {
    // V tile -> LDS, transposed: vt[d][key], d = 8grp + 32t + e, key = 16u + l16.
    // The tile is private to this wave; LDS operations of a wave complete in order.
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint4 vv = vr[buf][u][t];
        const uint32_t w4[4] = {vv.x, vv.y, vv.z, vv.w};
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
      s[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(dbf16x8_t, kr[buf][u][0]),
                                                     qb[0], df32x4_t{}, 0, 0, 0);
      s[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(dbf16x8_t, kr[buf][u][1]),
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
  };

  // This wave's tiles: wave, wave+4, wave+8, ... (the workgroup walks the chunk
  // front to back).  Every gload is unconditional, with the tile index clamped
  // to the last tile (a repeated tile is an L2 hit): the same number of loads
  // is then in flight on every path, and the compiler waits for one buffer
  // only (vmcnt(8)) instead of draining both.
  auto tile_kb = [&](int ti) { return k_begin + TK * min(ti, ntiles - 1); };
#pragma unroll
  for (int j = 0; j < NBUF; ++j) gload(j, tile_kb(wave + 4 * j));
  for (int ti = wave; ti < ntiles; ti += 4 * NBUF) {
#pragma unroll
    for (int j = 0; j < NBUF; ++j) {
      if (ti + 4 * j < ntiles) compute(j, k_begin + TK * (ti + 4 * j));
      gload(j, tile_kb(ti + 4 * j + 4 * NBUF));
    }
  }

  // o[dt][i] = O^T[d = 16dt + 4grp + i][head l16]; m is uniform over lane groups
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  float *red_o = reinterpret_cast<float *>(vt);  // [G][HD], this wave's V^T tile is done
  if (l16 < G) {
    if (grp == 0) {
      red_m[wave][l16] = m;
      red_l[wave][l16] = l;
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) red_o[l16 * HD + 16 * dt + 4 * grp + i] = o[dt][i];
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
      A += reinterpret_cast<const float *>(Vt[w2])[h * HD + d] * f;
    }
    float *part = p.ws + (((int64_t)b * p.n_heads + g * G + h) * p.n_split + split) * (HD + 2);
    part[2 + d] = A;
    if (d == 0) {
      part[0] = M * c;  // partials carry the max in the log2 domain
      part[1] = L;
    }
  }
}

// bf16 cache, n_kv_heads a multiple of 4: whole-row streaming version.
// A workgroup = (sequence, 4 consecutive KV heads, chunk).  Its 256 threads
// load each 32-key tile as 16-byte chunks of the 4 heads' 128-byte key rows
// (in a token-major cache one load instruction covers 1 KB: two token rows
// of the 4 heads, which streams HBM far better than per-head 64-byte
// pieces; other layouts reach each head's row through the head stride),
// into registers two tiles ahead, then write it row-major to LDS.  Wave w is KV head g0 + w:
// K fragments come from LDS with ds_read_b128, V^T fragments with the gfx950
// transpose read ds_read_b64_tr_b16, and the wave writes its own partials.
typedef short ds4_t __attribute__((ext_vector_type(4)));
constexpr int RKP = 4 * HD + 8;   // K tile row pitch (elements): 528 B, 16 rows hit 64 distinct banks
constexpr int RVP = 4 * HD + 16;  // V tile row pitch: 544 B, 4 rows x 32 B transpose reads conflict-free
constexpr int RCH = TK * 4 * HD * 2 / 16 / 256;  // 16-byte chunks per thread per array per tile

__device__ __forceinline__ dbf16x4_t lds_read_tr16(const bf16_t *p) {
  const ds4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) ds4_t *)(__attribute__((address_space(3))) void *)p);
  return __builtin_bit_cast(dbf16x4_t, r);
}

template <int G>
// register budget for 2 waves per SIMD (two register tiles ahead)
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void decode_bf16_rows_kernel(DecodeParams p) {
  // two tile buffers: one barrier per tile orders the LDS writes and reads
  __shared__ __attribute__((aligned(16))) bf16_t KL[2][TK * RKP];
  __shared__ __attribute__((aligned(16))) bf16_t VL[2][TK * RVP];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, grp = lane >> 4;
  const int hblocks = p.n_kv_heads >> 2;
  const int split = blockIdx.x % p.n_split;
  const int bh = blockIdx.x / p.n_split;
  const int b = bh / hblocks, g0 = (bh % hblocks) * 4;
  const int g = g0 + wave;

  int len = p.lens[b];
  len = len < 0 ? 0 : (len > p.max_len ? p.max_len : len);
  const int k_begin = split * p.chunk;
  if (k_begin >= len) return;  // the combine kernel ignores chunks past len
  const int k_end = min(k_begin + p.chunk, len);
  const int ntiles = (k_end - k_begin + TK - 1) / TK;

  const int64_t kv_rs = p.kv_rs;
  const bf16_t *Kr = (const bf16_t *)p.k + b * p.kv_bs + g0 * p.kv_hs;
  const bf16_t *Vr = (const bf16_t *)p.v + b * p.kv_bs + g0 * p.kv_hs;

  dbf16x8_t qb[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    if (l16 < G)
      qb[t] = *(const dbf16x8_t *)((const bf16_t *)p.q +
                                   ((int64_t)b * p.n_heads + g * G + l16) * HD + 8 * grp + 32 * t);
    else
      qb[t] = dbf16x8_t{};
  }

  // chunk c = tid + 256*i of a tile: row c / 32 (key), column (c % 32) * 8 elements.
  // Two register tiles (A, B) hold the next two tiles' K and V chunks.
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // native vector: stays in VGPRs
  struct RegTile {
    u32x4 k0, k1, k2, k3, v0, v1, v2, v3;
  };
  static_assert(RCH == 4, "register tile holds 4 chunks per array");
  const int crow = tid >> 5, ccol = (tid & 31) * 8;  // chunk i adds 8 rows
  const int64_t cofs = (ccol >> 6) * p.kv_hs + (ccol & 63);  // head ccol/64 of the four
  auto gload = [&](RegTile &r, int ti) __attribute__((always_inline)) {
    const int kb = k_begin + TK * min(ti, ntiles - 1);  // clamped: same load count on every path
    const int last = k_end - 1;  // past the end: a valid row, masked to P = 0
    const int64_t o0 = (int64_t)min(kb + crow, last) * kv_rs + cofs;
    const int64_t o1 = (int64_t)min(kb + crow + 8, last) * kv_rs + cofs;
    const int64_t o2 = (int64_t)min(kb + crow + 16, last) * kv_rs + cofs;
    const int64_t o3 = (int64_t)min(kb + crow + 24, last) * kv_rs + cofs;
    // streamed once: non-temporal loads
    r.k0 = __builtin_nontemporal_load((const u32x4 *)(Kr + o0)); r.v0 = __builtin_nontemporal_load((const u32x4 *)(Vr + o0));
    r.k1 = __builtin_nontemporal_load((const u32x4 *)(Kr + o1)); r.v1 = __builtin_nontemporal_load((const u32x4 *)(Vr + o1));
    r.k2 = __builtin_nontemporal_load((const u32x4 *)(Kr + o2)); r.v2 = __builtin_nontemporal_load((const u32x4 *)(Vr + o2));
    r.k3 = __builtin_nontemporal_load((const u32x4 *)(Kr + o3)); r.v3 = __builtin_nontemporal_load((const u32x4 *)(Vr + o3));
  };
  auto lstore = [&](const RegTile &r, int buf) __attribute__((always_inline)) {
    bf16_t *kd = KL[buf], *vd = VL[buf];
    *(u32x4 *)(kd + crow * RKP + ccol) = r.k0;
    *(u32x4 *)(kd + (crow + 8) * RKP + ccol) = r.k1;
    *(u32x4 *)(kd + (crow + 16) * RKP + ccol) = r.k2;
    *(u32x4 *)(kd + (crow + 24) * RKP + ccol) = r.k3;
    *(u32x4 *)(vd + crow * RVP + ccol) = r.v0;
    *(u32x4 *)(vd + (crow + 8) * RVP + ccol) = r.v1;
    *(u32x4 *)(vd + (crow + 16) * RVP + ccol) = r.v2;
    *(u32x4 *)(vd + (crow + 24) * RVP + ccol) = r.v3;
  };
  RegTile ta, tb;

  float m = -INFINITY, l = 0.f;
  df32x4_t o[4] = {df32x4_t{}, df32x4_t{}, df32x4_t{}, df32x4_t{}};
  const float c = p.c;
  auto compute = [&](int kb, int buf) __attribute__((always_inline)) {
    const bf16_t *kl = KL[buf] + wave * HD + 8 * grp;  // this wave's head inside the tile
    const bf16_t *vl = VL[buf] + wave * HD;
    df32x4_t s[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const bf16_t *kp = kl + (16 * u + l16) * RKP;
      s[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const dbf16x8_t *)(kp), qb[0], df32x4_t{},
                                                     0, 0, 0);
      s[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const dbf16x8_t *)(kp + 32), qb[1], s[u],
                                                     0, 0, 0);
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
    l = l * alpha + rs;
    m = m_new;
    // V^T operand: slot j of lane (grp, l16) = V[key 16(j/4) + 4grp + j%4][16dt + l16];
    // transpose read: local lane n supplies V[key 4grp + n/4 (+16)][16dt + 4(n%4) .. +3]
    const bf16_t *vp = vl + (4 * grp + (l16 >> 2)) * RVP + 4 * (l16 & 3);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      o[dt] *= alpha;
      const dbf16x4_t lo = lds_read_tr16(vp + 16 * dt);
      const dbf16x4_t hi = lds_read_tr16(vp + 16 * RVP + 16 * dt);
      const dbf16x8_t a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, o[dt], 0, 0, 0);
    }
  };

  // tile ti lives in LDS buffer ti & 1 and in register tile ta (even) / tb
  // (odd), loaded two tiles ahead.  Writing buffer x for tile t happens after
  // the barrier that follows the reads of tile t-2 (same buffer).
  gload(ta, 0);
  gload(tb, 1);
  lstore(ta, 0);
  gload(ta, 2);
  __syncthreads();
  for (int ti = 0; ti < ntiles; ti += 2) {
    compute(k_begin + TK * ti, 0);
    if (ti + 1 < ntiles) {  // workgroup-uniform
      lstore(tb, 1);
      gload(tb, ti + 3);
      __syncthreads();
      compute(k_begin + TK * (ti + 1), 1);
      lstore(ta, 0);
      gload(ta, ti + 4);
      __syncthreads();
    }
  }

  // o[dt][i] = O^T[d = 16dt + 4grp + i][query head g*G + l16]; m is uniform over lane groups
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (l16 < G) {
    float *part = p.ws + (((int64_t)b * p.n_heads + g * G + l16) * p.n_split + split) * (HD + 2);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) part[2 + 16 * dt + 4 * grp + i] = o[dt][i];
    if (grp == 0) {
      part[0] = m * c;  // log2 domain, as the other split kernels
      part[1] = l;
    }
  }
}

// bf16 cache, one workgroup per (sequence, KV head) over the whole cache:
// no partials in memory and no combine launch.  Chosen when there are at
// least as many (sequence, KV head) pairs as compute units, so every CU has a
// workgroup.  Wave w of the WWV takes the 32-key tiles w, w + WWV, ... and
// streams them through a private LDS tile (no workgroup barrier in the loop):
// 16-byte loads of the head's 128-byte cache rows, 8 rows per instruction,
// the next tile register-staged; the scores and P V on
// v_mfma_f32_16x16x32_bf16 as in the whole-row kernel.  The waves'
// (m, l, acc) are merged through LDS at the end and the workgroup writes the
// G output rows.  Four waves stream a cache (8 measured 8% slower on config
// 3, 2 3% slower).  When a KV head's rows are contiguous (row stride
// head_dim: a head-major cache) the workgroup has WWX waves and a cache more
// than 1.25x the batch's mean length uses all of them (once the other caches
// are done, one CU streams a long cache faster with more waves: config 3's
// ragged draw -4%, a few long caches among short ones -12%; uniform lengths
// keep four); token-major caches stream slower with more waves and keep four.
constexpr int WWV = 4;  // streaming waves per workgroup
constexpr int WWX = 6;  // waves of an adaptive whole-cache workgroup, active for a long cache
constexpr int kMeanBatchMax = 512;  // longer batches: four waves for every cache
constexpr int WKP = HD + 8;  // tile row pitch, 144 B: b128 K reads of 16 rows and tr16 V
                             // reads of 4 rows x 32 B hit distinct banks

// NW waves per workgroup: WWV, or WWX with the long-cache adaptation
template <int G, int NW>
__global__ __launch_bounds__(64 * NW) void decode_bf16_whole_kernel(DecodeParams p) {
  __shared__ __attribute__((aligned(16))) bf16_t KT[NW][TK * WKP];
  __shared__ __attribute__((aligned(16))) bf16_t VT[NW][TK * WKP];
  __shared__ float red_m[NW][G], red_l[NW][G];
  __shared__ float red_o[NW][G][HD];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, grp = lane >> 4;
  const int b = blockIdx.x / p.n_kv_heads, g = blockIdx.x % p.n_kv_heads;
  auto clamp_len = [&](int x) { return x < 0 ? 0 : (x > p.max_len ? p.max_len : x); };

  // the batch's total length (batches up to kMeanBatchMax sequences), summed
  // by every wave itself (no barrier), read with this sequence's length
  const bool adapt = NW > WWV && p.batch <= kMeanBatchMax;
  int part = 0;
  if (adapt)
    for (int i = lane; i < p.batch; i += 64) part += clamp_len(p.lens[i]);
  const int len = clamp_len(p.lens[b]);
  bf16_t *out = (bf16_t *)p.o + ((int64_t)b * p.n_heads + (int64_t)g * G) * HD;
  if (len == 0) {  // no key: zeros
    for (int idx = tid; idx < G * HD; idx += 64 * NW) out[idx] = f32_to_bf16(0.f);
    return;
  }
  int nw = WWV;  // streaming waves of this workgroup (uniform)
  if (adapt) {
#pragma unroll
    for (int o2 = 32; o2 > 0; o2 >>= 1) part += __shfl_xor(part, o2, 64);
    const int total = __builtin_amdgcn_readfirstlane(part);  // <= 512 * max_len
    if ((int64_t)len * p.batch * 4 > (int64_t)total * 5) nw = NW;
  }
  // wave w < nw takes the 32-key tiles w, w + nw, w + 2*nw, ...: the waves of
  // a workgroup stream adjacent tiles (a contiguous key range per wave, or the
  // KV heads of one sequence placed on one XCD, measured 3-4% slower)
  const int all_tiles = (len + TK - 1) / TK;
  const int kw0 = TK * wave, kw1 = len;
  const int tstride = TK * nw;  // keys between a wave's tiles
  const int ntiles = wave < nw && all_tiles > wave ? (all_tiles - wave + nw - 1) / nw : 0;

  const int64_t kv_rs = p.kv_rs;
  const bf16_t *Kr = (const bf16_t *)p.k + b * p.kv_bs + g * p.kv_hs;
  const bf16_t *Vr = (const bf16_t *)p.v + b * p.kv_bs + g * p.kv_hs;

  dbf16x8_t qb[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    if (l16 < G)
      qb[t] = *(const dbf16x8_t *)((const bf16_t *)p.q +
                                   ((int64_t)b * p.n_heads + g * G + l16) * HD + 8 * grp + 32 * t);
    else
      qb[t] = dbf16x8_t{};
  }

  // lane's 16-byte chunks of a tile: rows crow + 8i (i = 0..3), columns ccol..ccol+7
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  struct RegTile {
    u32x4 k0, k1, k2, k3, v0, v1, v2, v3;
  };
  const int crow = lane >> 3, ccol = (lane & 7) * 8;
  auto gload = [&](RegTile &r, int ti) __attribute__((always_inline)) {
    const int kb = kw0 + tstride * min(ti, ntiles - 1);  // clamped: same load count on every path
    const int last = min(kb + TK, kw1) - 1;  // past the end: a valid row, masked to P = 0
    const int64_t o0 = (int64_t)min(kb + crow, last) * kv_rs + ccol;
    const int64_t o1 = (int64_t)min(kb + crow + 8, last) * kv_rs + ccol;
    const int64_t o2 = (int64_t)min(kb + crow + 16, last) * kv_rs + ccol;
    const int64_t o3 = (int64_t)min(kb + crow + 24, last) * kv_rs + ccol;
    // streamed once: non-temporal loads
    r.k0 = __builtin_nontemporal_load((const u32x4 *)(Kr + o0)); r.v0 = __builtin_nontemporal_load((const u32x4 *)(Vr + o0));
    r.k1 = __builtin_nontemporal_load((const u32x4 *)(Kr + o1)); r.v1 = __builtin_nontemporal_load((const u32x4 *)(Vr + o1));
    r.k2 = __builtin_nontemporal_load((const u32x4 *)(Kr + o2)); r.v2 = __builtin_nontemporal_load((const u32x4 *)(Vr + o2));
    r.k3 = __builtin_nontemporal_load((const u32x4 *)(Kr + o3)); r.v3 = __builtin_nontemporal_load((const u32x4 *)(Vr + o3));
  };
  bf16_t *const kt = KT[wave], *const vt = VT[wave];
  auto lstore = [&](const RegTile &r) __attribute__((always_inline)) {
    *(u32x4 *)(kt + crow * WKP + ccol) = r.k0;
    *(u32x4 *)(kt + (crow + 8) * WKP + ccol) = r.k1;
    *(u32x4 *)(kt + (crow + 16) * WKP + ccol) = r.k2;
    *(u32x4 *)(kt + (crow + 24) * WKP + ccol) = r.k3;
    *(u32x4 *)(vt + crow * WKP + ccol) = r.v0;
    *(u32x4 *)(vt + (crow + 8) * WKP + ccol) = r.v1;
    *(u32x4 *)(vt + (crow + 16) * WKP + ccol) = r.v2;
    *(u32x4 *)(vt + (crow + 24) * WKP + ccol) = r.v3;
  };

  float m = -INFINITY, l = 0.f;
  df32x4_t o[4] = {df32x4_t{}, df32x4_t{}, df32x4_t{}, df32x4_t{}};
  const float c = p.c;
  // one 32-key tile from this wave's LDS tile; keys kb .. kb + 31
  auto compute = [&](int kb) __attribute__((always_inline)) {
    const bf16_t *kl = kt + 8 * grp;
    df32x4_t s[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const bf16_t *kp = kl + (16 * u + l16) * WKP;
      s[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const dbf16x8_t *)(kp), qb[0], df32x4_t{},
                                                     0, 0, 0);
      s[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const dbf16x8_t *)(kp + 32), qb[1], s[u],
                                                     0, 0, 0);
    }
    // s[u][i] = score of key kb + 16u + 4grp + i for query head g*G + l16
    if (kb + TK > kw1) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (kb + 16 * u + 4 * grp + i >= kw1) s[u][i] = -INFINITY;
    }
    float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                     fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m, mx);  // finite: every tile holds at least one key
    const float mc = m_new * c;
    const float alpha = __builtin_amdgcn_exp2f(m * c - mc);  // m = -inf -> 0
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
    l = l * alpha + rs;
    m = m_new;
    // V^T operand: slot j of lane (grp, l16) = V[key 16(j/4) + 4grp + j%4][16dt + l16];
    // transpose read: local lane n supplies V[key 4grp + n/4 (+16)][16dt + 4(n%4) .. +3]
    const bf16_t *vp = vt + (4 * grp + (l16 >> 2)) * WKP + 4 * (l16 & 3);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      o[dt] *= alpha;
      const dbf16x4_t lo = lds_read_tr16(vp + 16 * dt);
      const dbf16x4_t hi = lds_read_tr16(vp + 16 * WKP + 16 * dt);
      const dbf16x8_t a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, o[dt], 0, 0, 0);
    }
  };

  // The wave's tile ti goes through one register tile (loaded one tile ahead)
  // and the wave's LDS tile.  LDS instructions of one wave execute in order,
  // so a tile's writes follow the previous tile's reads (already consumed) and
  // precede its own reads with no barrier; wave_barrier keeps the compiler
  // from moving LDS accesses across.  One tile in flight per wave (4 KB of K
  // and of V; 32 KB per CU at 4 waves) streams best: two tiles ahead measured
  // 8% slower on config 3, more waves per workgroup slower still.
  if (ntiles > 0) {  // wave-uniform
    RegTile ta;
    gload(ta, 0);
    lstore(ta);
    gload(ta, 1);
    __builtin_amdgcn_wave_barrier();
    for (int ti = 0; ti < ntiles; ++ti) {
      compute(kw0 + tstride * ti);
      if (ti + 1 < ntiles) {
        __builtin_amdgcn_wave_barrier();
        lstore(ta);
        gload(ta, ti + 2);
        __builtin_amdgcn_wave_barrier();
      }
    }
  }

  // merge the waves: o[dt][i] = O^T[d = 16dt + 4grp + i][head g*G + l16]
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (l16 < G) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) red_o[wave][l16][16 * dt + 4 * grp + i] = o[dt][i];
    if (grp == 0) {
      red_m[wave][l16] = m * c;  // -inf for a wave without keys
      red_l[wave][l16] = l;
    }
  }
  __syncthreads();
  for (int idx = tid; idx < G * HD; idx += 64 * NW) {
    const int h = idx / HD, d = idx - h * HD;
    float M = red_m[0][h];
#pragma unroll
    for (int w = 1; w < NW; ++w) M = fmaxf(M, red_m[w][h]);  // finite: wave 0 has keys
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = __builtin_amdgcn_exp2f(red_m[w][h] - M);
      L += red_l[w][h] * wt;
      A += red_o[w][h][d] * wt;
    }
    out[idx] = f32_to_bf16(A / L);
  }
}

// Planned ragged decode (bn_gqa_decode_planned): the lengths are known on
// the host, which deals the batch's 32-key tiles -- units (sequence, KV head)
// in order -- into equal contiguous shares, one per workgroup and compute
// unit, so that every compute unit streams the same number of bytes and a
// long cache is cut across neighbouring workgroups instead of one compute
// unit streaming it alone after the others have finished.  A workgroup's
// share touches a few units (segments); its waves take the share's tiles in
// turn (tile i -> wave i % 4, the loads running on across segment
// boundaries), keep one (m, l, acc) per segment, and merge them through LDS
// at the end.  A unit lying wholly in the share is written directly.  A cut
// unit's head (its first tiles: the LAST segment of the share where it
// starts) merges it; every later part is the FIRST segment of its share, so
// its waves finish it early and hand their states to a fifth wave of the
// workgroup (through LDS and a workgroup counter), which merges them and
// writes the part's (m, l, acc) record to memory while the four stream on
// (written through to memory, a store holds up the wave that issued it, so
// none of the streaming waves issues one) -- every 64-bit word holding a
// value and this launch's epoch, so a reader knows a word is this launch's
// without any ordering between words, counters or waits.  At the end the
// head loads the records (one round trip: they were written while the rest
// of the shares streamed), merges and writes the output.  A record not yet this launch's
// is polled again a bounded number of times; past that the head streams the
// unit's remaining keys itself (never needed when the launch's workgroups
// run side by side, which 256 of them on 256 compute units do), so no
// workgroup waits on another without limit.
constexpr int kPlanBins = 256;   // workgroups of a planned launch, at most
constexpr int kPlanUnits = 256;  // (sequence, KV head) units, at most
constexpr int kPlanSeg = 8;      // units one share may touch, at most
constexpr int kPlanPolls = 1 << 14;  // re-polls of a record before the head streams the keys itself
// a part's record, G query heads: acc[G][HD], then m[G] (log2 units), l[G]
// (64-bit words; the writer wave's store instructions cover 512 contiguous bytes)
template <int G> constexpr int rec_words() { return G * HD + 2 * G; }

struct PlanParams {
  const void *q, *k, *v;
  void *o;
  uint64_t *rec;  // part records [record][rec_words<G>()], epoch in bits 32..63 of each word
  int batch, max_len, n_heads, n_kv_heads, n_units, share, total;  // share: sequence tiles per group
  float c;                         // scale * log2(e)
  uint32_t epoch;                  // this launch's tag (never 0; a fresh workspace may hold anything)
  int max_polls;                   // kPlanPolls; -1: ignore records, the heads stream every key
  int64_t kv_bs, kv_hs, kv_rs;     // cache strides (elements): sequence, KV head, key row
  uint32_t wg_start[kPlanBins];    // group: first sequence (bits 0..15), its first tile (16..31)
  uint32_t unit[kPlanUnits];       // record base (0..11), first group (12..23), parts (24..31)
  int32_t len[kPlanUnits];         // per sequence: length, clamped to [0, max_len]
};

// WWV streaming waves and one record-writer wave per workgroup
constexpr int kPlanThreads = 64 * (WWV + 1);

template <int G>
__global__ __launch_bounds__(kPlanThreads) void decode_bf16_planned_kernel(PlanParams p) {
  __shared__ __attribute__((aligned(16))) bf16_t KT[WWV][TK * WKP];
  __shared__ __attribute__((aligned(16))) bf16_t VT[WWV][TK * WKP];
  __shared__ float red_m[kPlanSeg][WWV][G], red_l[kPlanSeg][WWV][G];
  __shared__ float red_o[kPlanSeg][WWV][G][HD];
  __shared__ uint32_t seg0_done;  // streaming waves that have handed over segment 0

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool streamer = wave < WWV;  // wave WWV writes segment 0's record
  const int l16 = lane & 15, grp = lane >> 4;
  const int bin = blockIdx.x, Hkv = p.n_kv_heads;
  // workgroups come in groups of Hkv, one per KV head, that walk the same
  // share of the batch's sequences together (consecutive ids: dispatched at
  // the same time), so the KV heads' slices of a cache row are read close in
  // time, as in the whole-cache kernel
  const int grp_id = bin / Hkv, gh = bin - grp_id * Hkv;
  const int64_t kv_rs = p.kv_rs;
  auto tiles_of = [&](int b) { return (p.len[b] + TK - 1) / TK; };

  // units with no key at all: zeros, each written by workgroup u % gridDim.x
  for (int u = bin; u < p.n_units; u += gridDim.x) {
    if (p.len[u / Hkv] == 0) {
      bf16_t *out = (bf16_t *)p.o + ((int64_t)(u / Hkv) * p.n_heads + (int64_t)(u % Hkv) * G) * HD;
      for (int idx = tid; idx < G * HD; idx += kPlanThreads) out[idx] = f32_to_bf16(0.f);
    }
  }
  if (tid == 0) seg0_done = 0;
  __syncthreads();
  // This group's share [grp_id * share, +ntile) of the batch's sequence
  // tiles, as segments (one sequence each, sequences with keys in order) of
  // this workgroup's KV head.  Every wave walks them itself in scalar
  // registers -- no table, no barrier before the first loads -- forward only,
  // since a wave's tiles increase.
  const int ntile = min(p.share, p.total - grp_id * p.share);
  struct Seg {
    int s, b, end, kb0, len;  // sequence b; keys of local tile i: kb0 + 32 * i
    const bf16_t *kr, *vr;
  };
  auto seg_set = [&](Seg &x, int b, int lb, int t) __attribute__((always_inline)) {
    const int g = gh;
    x.b = b;
    x.len = p.len[b];
    x.end = min(ntile, lb + (x.len + TK - 1) / TK - t);
    x.kb0 = TK * (t - lb);
    x.kr = (const bf16_t *)p.k + b * p.kv_bs + g * p.kv_hs;
    x.vr = (const bf16_t *)p.v + b * p.kv_bs + g * p.kv_hs;
  };
  auto seg_first = [&](Seg &x) __attribute__((always_inline)) {
    x.s = 0;
    seg_set(x, (int)(p.wg_start[grp_id] & 0xffffu), 0, (int)(p.wg_start[grp_id] >> 16));
  };
  auto seg_next = [&](Seg &x) __attribute__((always_inline)) {
    int b = x.b + 1;
    while (b + 1 < p.batch && tiles_of(b) == 0) ++b;  // sequences without keys hold no tile
    ++x.s;
    seg_set(x, b, x.end, 0);
  };
  auto seg_adv = [&](Seg &x, int i) __attribute__((always_inline)) {
    while (i >= x.end && x.end < ntile) seg_next(x);
  };
  int nseg = 0;
  if (ntile > 0) {
    Seg x;
    seg_first(x);
    while (x.end < ntile && x.s + 1 < kPlanSeg) seg_next(x);
    nseg = x.s + 1;
  }

  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  struct RegTile {
    u32x4 k0, k1, k2, k3, v0, v1, v2, v3;
  };
  const int crow = lane >> 3, ccol = (lane & 7) * 8;
  auto gload = [&](RegTile &r, int i, const Seg &x) __attribute__((always_inline)) {
    const int kb = x.kb0 + TK * i, kw1 = x.len;
    const bf16_t *Kr = x.kr, *Vr = x.vr;
    const int last = min(kb + TK, kw1) - 1;  // past the end: a valid row, masked to P = 0
    const int64_t o0 = (int64_t)min(kb + crow, last) * kv_rs + ccol;
    const int64_t o1 = (int64_t)min(kb + crow + 8, last) * kv_rs + ccol;
    const int64_t o2 = (int64_t)min(kb + crow + 16, last) * kv_rs + ccol;
    const int64_t o3 = (int64_t)min(kb + crow + 24, last) * kv_rs + ccol;
    r.k0 = __builtin_nontemporal_load((const u32x4 *)(Kr + o0)); r.v0 = __builtin_nontemporal_load((const u32x4 *)(Vr + o0));
    r.k1 = __builtin_nontemporal_load((const u32x4 *)(Kr + o1)); r.v1 = __builtin_nontemporal_load((const u32x4 *)(Vr + o1));
    r.k2 = __builtin_nontemporal_load((const u32x4 *)(Kr + o2)); r.v2 = __builtin_nontemporal_load((const u32x4 *)(Vr + o2));
    r.k3 = __builtin_nontemporal_load((const u32x4 *)(Kr + o3)); r.v3 = __builtin_nontemporal_load((const u32x4 *)(Vr + o3));
  };
  // the query rows of a segment's unit: lane (grp, l16) holds head l16's
  // d = 8grp .. +7 and 32 + 8grp .. +7 (the MFMA B operand)
  auto gload_q = [&](dbf16x8_t (&qv)[2], const Seg &x) __attribute__((always_inline)) {
    const int b = x.b, g = gh;
#pragma unroll
    for (int t = 0; t < 2; ++t)
      qv[t] = l16 < G ? *(const dbf16x8_t *)((const bf16_t *)p.q +
                                            ((int64_t)b * p.n_heads + g * G + l16) * HD + 8 * grp + 32 * t)
                      : dbf16x8_t{};
  };
  // the writer wave (wave WWV) has no tile of its own and never uses these
  bf16_t *const kt = KT[streamer ? wave : 0], *const vt = VT[streamer ? wave : 0];
  auto lstore = [&](const RegTile &r) __attribute__((always_inline)) {
    *(u32x4 *)(kt + crow * WKP + ccol) = r.k0;
    *(u32x4 *)(kt + (crow + 8) * WKP + ccol) = r.k1;
    *(u32x4 *)(kt + (crow + 16) * WKP + ccol) = r.k2;
    *(u32x4 *)(kt + (crow + 24) * WKP + ccol) = r.k3;
    *(u32x4 *)(vt + crow * WKP + ccol) = r.v0;
    *(u32x4 *)(vt + (crow + 8) * WKP + ccol) = r.v1;
    *(u32x4 *)(vt + (crow + 16) * WKP + ccol) = r.v2;
    *(u32x4 *)(vt + (crow + 24) * WKP + ccol) = r.v3;
  };

  float m = -INFINITY, l = 0.f;
  df32x4_t o[4] = {df32x4_t{}, df32x4_t{}, df32x4_t{}, df32x4_t{}};
  dbf16x8_t qb[2], qn[2];
  const float c = p.c;
  // one 32-key tile from this wave's LDS tile: keys kb .. kb + 31 of a unit of kw1 keys
  auto compute = [&](int kb, int kw1) __attribute__((always_inline)) {
    const bf16_t *kl = kt + 8 * grp;
    df32x4_t s[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const bf16_t *kp = kl + (16 * u + l16) * WKP;
      s[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const dbf16x8_t *)(kp), qb[0], df32x4_t{},
                                                     0, 0, 0);
      s[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const dbf16x8_t *)(kp + 32), qb[1], s[u],
                                                     0, 0, 0);
    }
    if (kb + TK > kw1) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (kb + 16 * u + 4 * grp + i >= kw1) s[u][i] = -INFINITY;
    }
    float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                     fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m, mx);  // finite: every tile holds at least one key
    const float mc = m_new * c;
    const float alpha = __builtin_amdgcn_exp2f(m * c - mc);  // m = -inf -> 0
    float rs = 0.f;
    dbf16x8_t pb;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = __builtin_amdgcn_exp2f(fmaf(s[u][i], c, -mc));
        rs += e;
        pb[4 * u + i] = (__bf16)e;
      }
    l = l * alpha + rs;
    m = m_new;
    const bf16_t *vp = vt + (4 * grp + (l16 >> 2)) * WKP + 4 * (l16 & 3);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      o[dt] *= alpha;
      const dbf16x4_t lo = lds_read_tr16(vp + 16 * dt);
      const dbf16x4_t hi = lds_read_tr16(vp + 16 * WKP + 16 * dt);
      const dbf16x8_t a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, o[dt], 0, 0, 0);
    }
  };
  // segment 0 of the share is a later part of a cut unit (not its head):
  // every wave writes its state of it to the part's record as it moves on
  uint64_t *rec0 = nullptr;
  if (ntile > 0) {
    const int b0 = (int)(p.wg_start[grp_id] & 0xffffu);
    const uint32_t info0 = p.unit[b0 * Hkv + gh];
    const int parts0 = (int)(info0 >> 24), part0 = grp_id - (int)((info0 >> 12) & 0xfffu);
    if (parts0 > 1 && part0 > 0 && part0 < parts0)
      rec0 = p.rec + (int64_t)((info0 & 0xfffu) + part0) * rec_words<G>();
  }
  const uint64_t tag = (uint64_t)p.epoch << 32;
  auto put = [&](uint64_t *a, float v) __attribute__((always_inline)) {
    __hip_atomic_store(a, tag | __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
  };
  // this wave's state of segment s into LDS slot ls (o[dt][i] = O^T[16dt + 4grp + i][head l16])
  auto flush_to = [&](int s, int ls) __attribute__((always_inline)) {
    float lt = l + __shfl_xor(l, 16, 64);
    lt += __shfl_xor(lt, 32, 64);
    if (l16 < G) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) red_o[ls][wave][l16][16 * dt + 4 * grp + i] = o[dt][i];
      if (grp == 0) {
        red_m[ls][wave][l16] = m * c;  // -inf: no key of s in this wave
        red_l[ls][wave][l16] = lt;
      }
    }
    if (s == 0 && rec0) {  // segment 0 handed to the writer wave (LDS writes first)
      __builtin_amdgcn_wave_barrier();
      if (lane == 0) __hip_atomic_fetch_add(&seg0_done, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  };
  auto flush = [&](int s) __attribute__((always_inline)) { flush_to(s, s); };
  auto reset = [&]() __attribute__((always_inline)) {
    m = -INFINITY;
    l = 0.f;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = df32x4_t{};
  };

  // One register tile ahead per wave, as the whole-cache kernel: cur is the
  // segment of the tile computed, pre that of the tile in the registers;
  // when pre enters a new segment its query rows are loaded into qn, taken
  // over by qb when the wave's tiles reach that segment.
  int sc = -1;  // segment of the wave's running state
  if (streamer && wave < ntile) {  // wave-uniform
    Seg cur, pre;
    seg_first(cur);
    seg_adv(cur, wave);
    gload_q(qb, cur);
    RegTile ta;
    gload(ta, wave, cur);
    lstore(ta);
    pre = cur;
    if (wave + WWV < ntile) {
      seg_adv(pre, wave + WWV);
      if (pre.s != cur.s) gload_q(qn, pre);
      gload(ta, wave + WWV, pre);
    }
    __builtin_amdgcn_wave_barrier();
    for (int i = wave; i < ntile; i += WWV) {
      if (cur.s != sc) {  // a new segment: the previous one's state to LDS, a fresh state
        if (sc >= 0) flush(sc);
        for (int x = sc + 1; x < cur.s; ++x) {
          reset();
          flush(x);
        }
        reset();
        sc = cur.s;
      }
      compute(cur.kb0 + TK * i, cur.len);
      if (i + WWV < ntile) {
        __builtin_amdgcn_wave_barrier();
        lstore(ta);
        if (pre.s != cur.s) {
          qb[0] = qn[0];
          qb[1] = qn[1];
        }
        cur = pre;
        if (i + 2 * WWV < ntile) {
          const int s0 = pre.s;
          seg_adv(pre, i + 2 * WWV);
          if (pre.s != s0) gload_q(qn, pre);
          gload(ta, i + 2 * WWV, pre);
        }
        __builtin_amdgcn_wave_barrier();
      }
    }
  }
  if (streamer) {
    if (sc >= 0) flush(sc);
    reset();
    for (int x = sc + 1; x < nseg; ++x) flush(x);
  } else if (rec0) {
    // the writer wave: once the streaming waves have handed over segment 0
    // (bounded wait inside this workgroup; without the record the head
    // streams the keys itself), merge their states and write the record
    int polls = 0;
    while (__hip_atomic_load(&seg0_done, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < (uint32_t)WWV &&
           polls < kPlanPolls) {
      __builtin_amdgcn_s_sleep(2);
      ++polls;
    }
    if (polls < kPlanPolls) {
      for (int idx = lane; idx < G * HD; idx += 64) {
        const int h = idx / HD, d = idx - h * HD;
        float M = red_m[0][0][h];
#pragma unroll
        for (int w = 1; w < WWV; ++w) M = fmaxf(M, red_m[0][w][h]);
        float L = 0.f, A = 0.f;
#pragma unroll
        for (int w = 0; w < WWV; ++w) {
          const float wt = __builtin_amdgcn_exp2f(red_m[0][w][h] - M);
          L += red_l[0][w][h] * wt;
          A += red_o[0][w][h][d] * wt;
        }
        put(rec0 + idx, A);
        if (d == 0) {
          put(rec0 + G * HD + h, M);
          put(rec0 + G * HD + G + h, L);
        }
      }
    }
  }
  __syncthreads();

  // Merge the waves of each segment.  A unit wholly in this share is written.
  // A cut unit's later parts wrote their records from the waves (above); its
  // head -- the share's last segment -- loads them past the caches
  // (system-scope loads), each word tagged with this launch's epoch, merges
  // and writes the output.
  Seg x;
  if (nseg > 0) seg_first(x);
  for (int s = 0; s < nseg; ++s) {
    if (s > 0) seg_next(x);
    const int b = x.b, g = gh, u = b * Hkv + g;
    const uint32_t info = p.unit[u];
    const int parts = (int)(info >> 24), part = grp_id - (int)((info >> 12) & 0xfffu);
    if (parts > 1 && part != 0) continue;  // a later part: its record is written
    bf16_t *out = (bf16_t *)p.o + ((int64_t)b * p.n_heads + (int64_t)g * G) * HD;
    // this share's waves: (M, L, A) of output idx from LDS slot ls
    auto own = [&](int ls, int idx, float &M, float &L, float &A) __attribute__((always_inline)) {
      const int h = idx / HD, d = idx - h * HD;
      M = red_m[ls][0][h];
#pragma unroll
      for (int w = 1; w < WWV; ++w) M = fmaxf(M, red_m[ls][w][h]);
      L = 0.f;
      A = 0.f;
      if (M == -INFINITY) return;  // no key in any wave (a fallback slot can be empty)
#pragma unroll
      for (int w = 0; w < WWV; ++w) {
        const float wt = __builtin_amdgcn_exp2f(red_m[ls][w][h] - M);
        L += red_l[ls][w][h] * wt;
        A += red_o[ls][w][h][d] * wt;
      }
    };
    if (parts <= 1) {
      for (int idx = tid; idx < G * HD; idx += kPlanThreads) {
        float M, L, A;
        own(s, idx, M, L, A);
        out[idx] = f32_to_bf16(A / L);
      }
      continue;
    }
    // the head of a cut unit: this share holds its first tiles, the later
    // parts the rest; each thread merges its outputs from its own loads
    constexpr int NO = (G * HD + kPlanThreads - 1) / kPlanThreads;  // outputs per thread
    const uint64_t *recb = p.rec + (int64_t)(info & 0xfffu) * rec_words<G>();
    float Mv[NO], Lv[NO], Av[NO];
    bool ok = true;
    auto gather = [&]() __attribute__((always_inline)) {
      ok = true;
#pragma unroll
      for (int j = 0; j < NO; ++j) {
        const int idx = min(tid + kPlanThreads * j, G * HD - 1);  // past G*HD: a repeat, not stored
        own(s, idx, Mv[j], Lv[j], Av[j]);
      }
      // one part at a time, every word of the part requested before any is
      // used: one round trip per later part
      for (int q = 1; q < parts; ++q) {
        const uint64_t *r = recb + (int64_t)q * rec_words<G>();
        uint64_t wm[NO], wl[NO], wa[NO];
#pragma unroll
        for (int j = 0; j < NO; ++j) {
          const int idx = min(tid + kPlanThreads * j, G * HD - 1);
          const int h = idx / HD;
          wm[j] = __hip_atomic_load(r + G * HD + h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
          wl[j] = __hip_atomic_load(r + G * HD + G + h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
          wa[j] = __hip_atomic_load(r + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
#pragma unroll
        for (int j = 0; j < NO; ++j) {
          ok = ok && (wm[j] >> 32) == p.epoch && (wl[j] >> 32) == p.epoch && (wa[j] >> 32) == p.epoch;
          const float mq = __builtin_bit_cast(float, (uint32_t)wm[j]);
          const float m2 = fmaxf(Mv[j], mq);  // finite: this share's part has keys
          const float a1 = __builtin_amdgcn_exp2f(Mv[j] - m2), a2 = __builtin_amdgcn_exp2f(mq - m2);
          Lv[j] = Lv[j] * a1 + __builtin_bit_cast(float, (uint32_t)wl[j]) * a2;
          Av[j] = Av[j] * a1 + __builtin_bit_cast(float, (uint32_t)wa[j]) * a2;
          Mv[j] = m2;
        }
      }
    };
    bool all_ok = false;
    if (p.max_polls >= 0) {
      gather();
      all_ok = __syncthreads_and(ok);
      for (int poll = 0; !all_ok && poll < p.max_polls; ++poll) {
        __builtin_amdgcn_s_sleep(4);
        gather();
        all_ok = __syncthreads_and(ok);
      }
    }
    if (!all_ok) {
      // Fallback: stream the unit's keys past this share's tiles here, into a
      // free LDS slot (slot 0 is finished when s > 0; slot 1 is unused when
      // the share holds this segment only), and merge with this share's part.
      const int ls = s == 0 ? 1 : 0;
      // local tile i of x holds keys x.kb0 + 32 i, so the later parts start
      // at the unit's tile x.kb0 / 32 + x.end
      const int first_rest = x.kb0 / TK + x.end;
      const int rest = tiles_of(b) - first_rest;
      Seg y = x;
      y.kb0 = TK * first_rest;  // local tile i of y: keys kb0 + 32 i
      if (streamer) {
        reset();
        if (wave < rest) {
          dbf16x8_t qf[2];
          gload_q(qf, y);
          qb[0] = qf[0];
          qb[1] = qf[1];
          for (int i = wave; i < rest; i += WWV) {
            RegTile r;
            gload(r, i, y);
            __builtin_amdgcn_wave_barrier();
            lstore(r);
            __builtin_amdgcn_wave_barrier();
            compute(y.kb0 + TK * i, y.len);
            __builtin_amdgcn_wave_barrier();
          }
        }
        flush_to(-1, ls);
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < NO; ++j) {
        const int idx = min(tid + kPlanThreads * j, G * HD - 1);
        float M, L, A, M2, L2, A2;
        own(s, idx, M, L, A);
        own(ls, idx, M2, L2, A2);
        const float mm = fmaxf(M, M2);
        const float a1 = __builtin_amdgcn_exp2f(M - mm), a2 = __builtin_amdgcn_exp2f(M2 - mm);
        Mv[j] = mm;
        Lv[j] = L * a1 + L2 * a2;
        Av[j] = A * a1 + A2 * a2;
      }
    }
#pragma unroll
    for (int j = 0; j < NO; ++j) {
      const int idx = tid + kPlanThreads * j;
      if (idx < G * HD) out[idx] = f32_to_bf16(Av[j] / Lv[j]);
    }
    __syncthreads();  // the fallback's LDS slot and state are reused by the next segment
  }
}

// One thread per (b, head, d): merge the chunks [0, ceil(len/chunk)) in one
// pass (running log-sum-exp), four chunks' loads in flight at a time.
template <typename T>
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeParams p) {
  // one thread per 4 consecutive d of one (sequence, head); the partial loads
  // of 8 chunks are issued together with the length load (slots past the
  // valid chunks read an in-range record and are skipped in the merge).
  // chunk 0: the short-cache split's chunk, derived from the length.
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)p.batch * p.n_heads * (HD / 4)) return;
  const int d0 = (int)(idx % (HD / 4)) * 4;
  const int64_t bh = idx / (HD / 4);
  const int b = (int)(bh / p.n_heads);
  const float *part = p.ws + bh * p.n_split * kDecRec;
  DecMerge mg;
  int len = p.hlen >= 0 ? p.hlen : p.lens[b];
  mg.load8(part, p.n_split, 0, d0);
  len = len < 0 ? 0 : (len > p.max_len ? p.max_len : len);
  const int chunk = p.chunk > 0 ? p.chunk : short_split_chunk(len, p.n_split);
  const int nvalid = (len + chunk - 1) / chunk;  // chunks holding keys (finite max)
  mg.start();
  mg.merge8(0, nvalid);  // the first 8 chunks need no branch on the length
  for (int s0 = 8; s0 < nvalid; s0 += 8) {
    mg.load8(part, p.n_split, s0, d0);
    mg.merge8(s0, nvalid);
  }
  const float4 r = mg.result();
  T *out = (T *)p.o + bh * HD + d0;
  Elem<T>::store(out + 0, r.x);
  Elem<T>::store(out + 1, r.y);
  Elem<T>::store(out + 2, r.z);
  Elem<T>::store(out + 3, r.w);
}

// split-K workgroup targets: per-head kernels / whole-row kernel (4 KV heads
// per workgroup)
constexpr int kMinWg = 2048, kRowsMinWg = 512;
int choose_chunk(int batch, int max_len, int units, int min_wg) {
  // enough workgroups to cover the 256 CUs several times over (a partial last
  // round of resident workgroups costs a whole round), chunks >= 128 keys
  int chunk = 1024;
  while (chunk > 128 && (int64_t)batch * units * ((max_len + chunk - 1) / chunk) < min_wg)
    chunk >>= 1;
  return chunk;
}

template <typename T, int G>
void launch_split(const DecodeParams &p, dim3 grid, hipStream_t s) {
  if constexpr (std::is_same<T, bf16_t>::value) {
    if (p.n_kv_heads % 4 == 0)
      hipLaunchKernelGGL((decode_bf16_rows_kernel<G>), grid, dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((decode_bf16_mfma_kernel<G>), grid, dim3(256), 0, s, p);
  } else {
    hipLaunchKernelGGL((decode_split_kernel<T, G, 4, DEC_SPLIT>), grid, dim3(256), 0, s, p);
  }
}

bool rows_path(const DecodeParams &p, bool bf16) { return bf16 && p.n_kv_heads % 4 == 0; }



void launch_short(const DecodeParams &p, hipStream_t s) {
  const dim3 grid((unsigned)((int64_t)p.batch * p.n_heads / kShortG * p.n_split));
  hipLaunchKernelGGL((decode_split_kernel<float, kShortG, kShortWV, DEC_SHORT>), grid, dim3(64 * kShortWV),
                     0, s, p);
}

template <typename T>
int launch_decode(const DecodeParams &p, int G, hipStream_t s) {
  const bool rows = rows_path(p, std::is_same<T, bf16_t>::value);
  const dim3 grid((unsigned)((int64_t)p.batch * (rows ? p.n_kv_heads / 4 : p.n_kv_heads) *
                             p.n_split));
  switch (G) {
    case 0: launch_short(p, s); break;  // short-cache split (fp32)
    case 1: launch_split<T, 1>(p, grid, s); break;
    case 2: launch_split<T, 2>(p, grid, s); break;
    case 4: launch_split<T, 4>(p, grid, s); break;
    default: launch_split<T, 8>(p, grid, s); break;
  }
  BN_LAUNCH_CHECK();
  const int64_t n = (int64_t)p.batch * p.n_heads * (HD / 4);
  hipLaunchKernelGGL(decode_combine_kernel<T>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     s, p);
  BN_LAUNCH_CHECK();
  return BN_OK;
}

}  // namespace

bool short_path_ok(int dtype, int batch, int max_len, int n_heads) {
  return dtype == BN_F32 && batch > 0 && max_len > 0 && max_len <= kShortMaxLen &&
         (int64_t)batch * n_heads <= kShortMaxUnits;
}

int decode_short_partials(const float *q, const float *k_cache, const float *v_cache,
                          const int32_t *seq_lens, int host_len, float *part, int batch, int max_len,
                          int n_heads, int n_kv_heads, float scale, hipStream_t s) {
  DecodeParams p;
  p.q = q; p.k = k_cache; p.v = v_cache; p.lens = seq_lens; p.o = nullptr; p.ws = part;
  p.hlen = host_len;
  p.batch = batch; p.max_len = max_len; p.n_heads = n_heads; p.n_kv_heads = n_kv_heads;
  p.kv_rs = (int64_t)n_kv_heads * HD;  // contiguous [batch, max_len, n_kv_heads, 64]
  p.kv_hs = HD;
  p.kv_bs = (int64_t)max_len * p.kv_rs;
  p.n_split = kShortSplits;
  p.chunk = 0;
  p.c = scale * 1.4426950408889634f;
  launch_short(p, s);
  BN_LAUNCH_CHECK();
  return BN_OK;
}

// Device address of `scratch` per device, looked up once per device by
// bn_init (with that device current).  Each GPU holds its own copy of the
// array at its own address.
constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kMaxScratchDevices];

// the planned decode's launch epochs (the tag of every record word a launch
// writes; never 0)
static std::atomic<uint32_t> g_plan_epoch{0};
static void *g_short_cnt_ptr[kMaxScratchDevices];
static std::atomic<uint32_t> g_short_next{0};

int decode_scratch_setup(int device) {
  if (device < 0 || device >= kMaxScratchDevices)
    return fail(BN_ERR_UNSUPPORTED, "bn_init: device " + std::to_string(device) +
                                        " above the decode scratch table (" +
                                        std::to_string(kMaxScratchDevices) + " devices)");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[device]) return BN_OK;
  void *ptr = nullptr;
  BN_HIP_TRY(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
  if (!ptr) return fail(BN_ERR_HIP, "bn_init: decode scratch has no device address");
  void *scnt = nullptr;  // the short-cache decode's split counters
  BN_HIP_TRY(hipGetSymbolAddress(&scnt, HIP_SYMBOL(short_counters)));
  if (!scnt) return fail(BN_ERR_HIP, "bn_init: short decode counters have no device address");
  g_scratch_ptr[device] = ptr;
  g_short_cnt_ptr[device] = scnt;
  return BN_OK;
}

namespace {
void *decode_scratch(int device) {
  if (device < 0 || device >= kMaxScratchDevices) return nullptr;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  return g_scratch_ptr[device];
}
// the next planned-decode launch epoch (never 0)
uint32_t next_plan_epoch() {
  uint32_t e = g_plan_epoch.fetch_add(1) + 1;
  if (e == 0) e = g_plan_epoch.fetch_add(1) + 1;
  return e;
}
// the next counter slot of the short-cache decode on `device` (null: not set up)
constexpr int kShortSlots = 16;
static_assert(kShortSlots * kShortMaxUnits == 16 * 256, "short_counters holds kShortSlots slots");
uint32_t *short_counter_slot(int device) {
  if (device < 0 || device >= kMaxScratchDevices) return nullptr;
  void *base;
  {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    base = g_short_cnt_ptr[device];
  }
  if (!base) return nullptr;
  return (uint32_t *)base + (g_short_next.fetch_add(1) % kShortSlots) * kShortMaxUnits;
}
}  // namespace
}  // namespace bn

using namespace bn;

extern "C" {

size_t bn_gqa_decode_workspace_size(int batch, int max_len, int n_heads, int head_dim) {
  if (batch <= 0 || max_len <= 0 || n_heads <= 0 || head_dim != HD) return 0;
  // n_split does not depend on n_kv_heads by more than the chunk choice; size
  // for the smallest chunk (most splits) so any n_kv_heads fits
  int64_t n_split = (max_len + 127) / 128;
  if (short_path_ok(BN_F32, batch, max_len, n_heads)) n_split = std::max<int64_t>(n_split, kShortSplits);
  return (size_t)batch * n_heads * n_split * kDecRec * sizeof(float);
}

}  // extern "C"

namespace bn {
namespace {
// bn_gqa_decode and bn_gqa_decode_noalloc: the same validation, kernels and
// launch shapes; they differ only in where the split-K partials live (the
// caller's workspace or the pool, against the file-scope scratch array).
// strides: the caches' element strides (sequence, KV head, key row), or null
// for a contiguous [batch, max_len, n_kv_heads, head_dim] cache.
int gqa_decode_impl(int dtype, const void *q, const void *k_cache, const void *v_cache,
                    const int32_t *seq_lens, void *o, int batch, int max_len, int n_heads,
                    int n_kv_heads, int head_dim, float scale, void *workspace,
                    size_t workspace_bytes, bool noalloc, void *stream,
                    const int64_t *strides = nullptr) {
  const char *op = noalloc ? "GQA decode (no allocation)" : strides ? "GQA decode (strided)" : "GQA decode";
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
  if (strides) {
    // every key row starts 16-byte aligned (the kernels load 16 bytes per lane)
    const int64_t align = dtype == BN_BF16 ? 8 : 4;
    for (int i = 0; i < 3; ++i)
      if (strides[i] <= 0 || strides[i] % align != 0 || strides[i] > ((int64_t)1 << 40))
        return fail(BN_ERR_INVALID_ARG, std::string(op) + ": cache strides must be positive multiples of " +
                                            std::to_string(align) + " elements (16 bytes)");
  }
  if (!q || !k_cache || !v_cache || !seq_lens || !o)
    return fail(BN_ERR_INVALID_ARG, std::string(op) + ": NULL pointer");
  if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15u)
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": q and caches must be 16-byte aligned");
  // a caller's workspace must hold what bn_gqa_decode_workspace_size() asks
  // for, whichever kernel the call takes (checked before any device work)
  if (workspace) {
    const size_t want = bn_gqa_decode_workspace_size(batch, max_len, n_heads, head_dim);
    if (workspace_bytes < want)
      return fail(BN_ERR_INVALID_ARG, std::string(op) + ": workspace of " +
                                          std::to_string(workspace_bytes) + " bytes, need " +
                                          std::to_string(want));
  }
  DecodeParams p;
  p.q = q; p.k = k_cache; p.v = v_cache; p.lens = seq_lens; p.o = o;
  p.batch = batch; p.max_len = max_len; p.n_heads = n_heads; p.n_kv_heads = n_kv_heads;
  p.kv_bs = strides ? strides[0] : (int64_t)max_len * n_kv_heads * HD;
  p.kv_hs = strides ? strides[1] : HD;
  p.kv_rs = strides ? strides[2] : (int64_t)n_kv_heads * HD;
  const bool short_split = short_path_ok(dtype, batch, max_len, n_heads);
  if (!short_split && dtype == BN_BF16) {  // one workgroup per (sequence, KV head) when that fills the CUs
    int st = ensure_device();
    if (st) return st;
    const int cus = device_cu_count();
    if (cus > 0 && (int64_t)batch * n_kv_heads >= cus) {
      p.ws = nullptr;
      p.n_split = 1;
      p.chunk = max_len;
      p.c = scale * 1.4426950408889634f;
      hipStream_t s = as_stream(stream);
      // a KV head's rows contiguous: long caches may take more waves
      const bool wide = p.kv_rs == HD && batch <= kMeanBatchMax;
      const dim3 grid((unsigned)((int64_t)batch * n_kv_heads)), block(64 * (wide ? WWX : WWV));
#define BN_WHOLE(GG)                                                                        \
  do {                                                                                      \
    if (wide)                                                                               \
      hipLaunchKernelGGL((decode_bf16_whole_kernel<GG, WWX>), grid, block, 0, s, p);        \
    else                                                                                    \
      hipLaunchKernelGGL((decode_bf16_whole_kernel<GG, WWV>), grid, block, 0, s, p);        \
  } while (0)
      switch (G) {
        case 1: BN_WHOLE(1); break;
        case 2: BN_WHOLE(2); break;
        case 4: BN_WHOLE(4); break;
        default: BN_WHOLE(8); break;
      }
#undef BN_WHOLE
      BN_LAUNCH_CHECK();
      return BN_OK;
    }
  }
  if (short_split) {  // kShortSplits splits of the length; the combine derives the chunk
    p.chunk = 0;
    p.n_split = kShortSplits;
  } else {
    // the whole-row kernel gives each workgroup 4 KV heads: 1/4 of the workgroups per chunk
    p.chunk = rows_path(p, dtype == BN_BF16)
                  ? choose_chunk(batch, max_len, n_kv_heads / 4, kRowsMinWg)
                  : choose_chunk(batch, max_len, n_kv_heads, kMinWg);
    p.n_split = (max_len + p.chunk - 1) / p.chunk;
  }
  p.c = scale * 1.4426950408889634f;
  const size_t need = (size_t)batch * n_heads * p.n_split * (HD + 2) * sizeof(float);
  if (noalloc && need > (size_t)BN_GQA_DECODE_SCRATCH_BYTES)
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": the call needs " + std::to_string(need) +
                                        " bytes of chunk partials, above the " +
                                        std::to_string((size_t)BN_GQA_DECODE_SCRATCH_BYTES) +
                                        "-byte scratch");
  int st = ensure_device();
  if (st) return st;
  hipStream_t s = as_stream(stream);
  void *ws = workspace;
  bool own = false;
  if (noalloc) {
    // every record the combine reads is written by this call's split kernel
    // first, so the scratch needs no clearing
    ws = decode_scratch(library_device());
    if (!ws) return fail(BN_ERR_HIP, std::string(op) + ": scratch address not set up for device " +
                                         std::to_string(library_device()));
  } else if (!ws) {
    if ((st = bn_alloc(&ws, need, stream))) return st;
    own = true;
  }
  p.ws = (float *)ws;
  if (short_split) {  // one launch: the unit's last split merges its records
    p.cnt = short_counter_slot(library_device());
    if (!p.cnt) {
      st = fail(BN_ERR_HIP, std::string(op) + ": split counters not set up for device " +
                                std::to_string(library_device()));
    } else {
      launch_short(p, s);
      const hipError_t e = hipGetLastError();
      st = e == hipSuccess ? BN_OK : hip_fail(e, __FILE__, __LINE__);
    }
  } else {
    st = dtype == BN_BF16 ? launch_decode<bf16_t>(p, G, s) : launch_decode<float>(p, G, s);
  }
  if (own) {
    int st2 = bn_free(ws, stream);
    if (st == BN_OK) st = st2;
  }
  return st;
}
// The planned launch's share plan from the host lengths: groups of
// n_kv_heads workgroups (one per KV head) split the batch's sequence tiles
// into equal contiguous shares.  False when the batch is not worth planning
// (longest sequence within 1.25x of the mean: the whole-cache kernel is
// balanced already) or does not fit the plan's limits.
bool build_plan(const int32_t *h_lens, int batch, int max_len, int n_kv_heads, int n_heads, int cus,
                PlanParams &pl, int &bins, int &records) {
  (void)n_heads;
  const int units = batch * n_kv_heads;
  if (units > kPlanUnits || batch > kPlanUnits || cus <= 0) return false;
  std::vector<int> tiles(batch);
  int64_t total = 0;
  int tmax = 0;
  for (int b = 0; b < batch; ++b) {
    const int len = h_lens[b] < 0 ? 0 : (h_lens[b] > max_len ? max_len : h_lens[b]);
    pl.len[b] = len;
    tiles[b] = (len + TK - 1) / TK;
    total += tiles[b];
    tmax = std::max(tmax, tiles[b]);
  }
  if (total == 0 || total > 0xffffff || (int64_t)tmax * batch * 4 <= total * 5) return false;
  const int groups0 = (int)std::min<int64_t>(std::min(cus, kPlanBins) / n_kv_heads, total);
  if (groups0 <= 0) return false;
  const int share = (int)((total + groups0 - 1) / groups0);
  const int groups = (int)((total + share - 1) / share);
  bins = groups * n_kv_heads;
  if (share > 0xffff || tmax > 0xffff) return false;
  // prefix of each sequence's tiles; group k takes tiles [k*share, (k+1)*share)
  std::vector<int64_t> pre(batch + 1, 0);
  for (int b = 0; b < batch; ++b) pre[b + 1] = pre[b] + tiles[b];
  int b = 0;
  for (int k = 0; k < groups; ++k) {
    const int64_t g0 = (int64_t)k * share;
    while (b < batch && pre[b] + tiles[b] <= g0) ++b;  // skips empty sequences
    pl.wg_start[k] = (uint32_t)b | ((uint32_t)(g0 - pre[b]) << 16);
    // the sequences this share touches (with keys), at most kPlanSeg
    int n = 0;
    for (int v = b; v < batch && pre[v] < g0 + share; ++v) n += tiles[v] > 0;
    if (n > kPlanSeg) return false;
  }
  records = 0;
  for (int v = 0; v < batch; ++v) {
    int c0 = 0, parts = 1;
    if (tiles[v] > 0) {
      c0 = (int)(pre[v] / share);
      parts = (int)((pre[v] + tiles[v] - 1) / share) - c0 + 1;
    }
    for (int g = 0; g < n_kv_heads; ++g) {  // each KV head's unit: parts in the same groups
      const int base = parts > 1 ? records : 0;
      if (parts > 1) records += parts;
      if (records > 0xfff || c0 > 0xfff || parts > 0xff) return false;
      pl.unit[v * n_kv_heads + g] = (uint32_t)base | ((uint32_t)c0 << 12) | ((uint32_t)parts << 24);
    }
  }
  pl.share = share;
  pl.total = (int)total;
  pl.n_units = units;
  return true;
}
}  // namespace
}  // namespace bn

extern "C" {

int bn_gqa_decode(int dtype, const void *q, const void *k_cache, const void *v_cache,
                  const int32_t *seq_lens, void *o, int batch, int max_len, int n_heads,
                  int n_kv_heads, int head_dim, float scale, void *workspace,
                  size_t workspace_bytes, void *stream) {
  return gqa_decode_impl(dtype, q, k_cache, v_cache, seq_lens, o, batch, max_len, n_heads,
                         n_kv_heads, head_dim, scale, workspace, workspace_bytes, false, stream);
}

int bn_gqa_decode_noalloc(int dtype, const void *q, const void *k_cache, const void *v_cache,
                          const int32_t *seq_lens, void *o, int batch, int max_len, int n_heads,
                          int n_kv_heads, int head_dim, float scale, void *stream) {
  return gqa_decode_impl(dtype, q, k_cache, v_cache, seq_lens, o, batch, max_len, n_heads,
                         n_kv_heads, head_dim, scale, nullptr, 0, true, stream);
}

int bn_gqa_decode_strided(int dtype, const void *q, const void *k_cache, const void *v_cache,
                          const int32_t *seq_lens, void *o, int batch, int max_len, int n_heads,
                          int n_kv_heads, int head_dim, int64_t cache_seq_stride,
                          int64_t cache_head_stride, int64_t cache_row_stride, float scale,
                          void *workspace, size_t workspace_bytes, void *stream) {
  const int64_t strides[3] = {cache_seq_stride, cache_head_stride, cache_row_stride};
  return gqa_decode_impl(dtype, q, k_cache, v_cache, seq_lens, o, batch, max_len, n_heads,
                         n_kv_heads, head_dim, scale, workspace, workspace_bytes, false, stream,
                         strides);
}

size_t bn_gqa_decode_planned_workspace_size(int batch, int max_len, int n_heads, int n_kv_heads,
                                            int head_dim) {
  if (batch <= 0 || max_len <= 0 || n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads ||
      head_dim != HD)
    return 0;
  // the unplanned fallback's partials, or the plan's part records (at most
  // one per unit plus one per workgroup boundary; each holds every wave's
  // state as epoch-tagged 64-bit words)
  const size_t recs = ((size_t)batch * n_kv_heads + kPlanBins) *
                      ((size_t)(n_heads / n_kv_heads) * HD + 2 * (n_heads / n_kv_heads)) * sizeof(uint64_t);
  return std::max(bn_gqa_decode_workspace_size(batch, max_len, n_heads, head_dim), recs);
}

}  // extern "C"

namespace bn {
namespace {
// bn_gqa_decode_planned and bn_gqa_decode_planned_strided (strides: null for
// a contiguous [batch, max_len, n_kv_heads, 64] cache)
int gqa_decode_planned_impl(int dtype, const void *q, const void *k_cache, const void *v_cache,
                            const int32_t *seq_lens, const int32_t *h_seq_lens, void *o, int batch,
                            int max_len, int n_heads, int n_kv_heads, int head_dim, float scale,
                            void *workspace, size_t workspace_bytes, void *stream,
                            const int64_t *strides) {
  const char *op = "GQA decode (planned)";
  if (batch > 0 && !h_seq_lens)
    return fail(BN_ERR_INVALID_ARG, std::string(op) + ": NULL host lengths");
  if (workspace && batch > 0) {
    const size_t want = bn_gqa_decode_planned_workspace_size(batch, max_len, n_heads, n_kv_heads, head_dim);
    if (want && workspace_bytes < want)
      return fail(BN_ERR_INVALID_ARG, std::string(op) + ": workspace of " +
                                          std::to_string(workspace_bytes) + " bytes, need " +
                                          std::to_string(want));
  }
  // the plan applies to bf16 caches of 1, 2, 4 or 8 query heads per KV head
  // with at least as many units as compute units; anything else (and every
  // argument check) is bn_gqa_decode's
  const int G = n_kv_heads > 0 ? n_heads / n_kv_heads : 0;
  bool planned = dtype == BN_BF16 && head_dim == HD && batch > 0 && max_len > 0 && n_kv_heads > 0 &&
                 n_heads % n_kv_heads == 0 && (G == 1 || G == 2 || G == 4 || G == 8) &&
                 (scale > 0.f) && std::isfinite(scale) && q && k_cache && v_cache && seq_lens && o &&
                 !(((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15u);
  if (strides)
    for (int i = 0; i < 3; ++i)
      planned = planned && strides[i] > 0 && strides[i] % 8 == 0 && strides[i] <= ((int64_t)1 << 40);
  int st;
  PlanParams pl;
  int bins = 0, records = 0;
  if (planned) {
    if ((st = ensure_device())) return st;
    const int cus = device_cu_count();
    planned = (int64_t)batch * n_kv_heads >= cus &&
              build_plan(h_seq_lens, batch, max_len, n_kv_heads, n_heads, cus, pl, bins, records);
  }
  if (!planned)
    return gqa_decode_impl(dtype, q, k_cache, v_cache, seq_lens, o, batch, max_len, n_heads, n_kv_heads,
                           head_dim, scale, workspace, workspace_bytes, false, stream, strides);
  pl.q = q; pl.k = k_cache; pl.v = v_cache; pl.o = o;
  pl.batch = batch; pl.max_len = max_len; pl.n_heads = n_heads; pl.n_kv_heads = n_kv_heads;
  pl.kv_bs = strides ? strides[0] : (int64_t)max_len * n_kv_heads * HD;
  pl.kv_hs = strides ? strides[1] : HD;
  pl.kv_rs = strides ? strides[2] : (int64_t)n_kv_heads * HD;
  pl.c = scale * 1.4426950408889634f;
  pl.epoch = next_plan_epoch();
  // BN_PLAN_FALLBACK=1 (tests): the heads ignore the records and stream the
  // later parts' keys themselves -- the path a head takes if a record never
  // arrives
  const char *fb = std::getenv("BN_PLAN_FALLBACK");
  pl.max_polls = (fb && fb[0] == '1') ? -1 : kPlanPolls;
  hipStream_t s = as_stream(stream);
  void *ws = workspace;
  bool own = false;
  const size_t need = (size_t)std::max(records, 1) * ((size_t)G * HD + 2 * G) * sizeof(uint64_t);
  if (!ws && records > 0) {
    if ((st = bn_alloc(&ws, need, stream))) return st;
    own = true;
  }
  pl.rec = (uint64_t *)ws;
  const dim3 grid((unsigned)bins), block(kPlanThreads);
  switch (G) {
    case 1: hipLaunchKernelGGL(decode_bf16_planned_kernel<1>, grid, block, 0, s, pl); break;
    case 2: hipLaunchKernelGGL(decode_bf16_planned_kernel<2>, grid, block, 0, s, pl); break;
    case 4: hipLaunchKernelGGL(decode_bf16_planned_kernel<4>, grid, block, 0, s, pl); break;
    default: hipLaunchKernelGGL(decode_bf16_planned_kernel<8>, grid, block, 0, s, pl); break;
  }
  st = BN_OK;
  {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) st = hip_fail(e, __FILE__, __LINE__);
  }
  if (own) {
    int st2 = bn_free(ws, stream);
    if (st == BN_OK) st = st2;
  }
  return st;
}
}  // namespace
}  // namespace bn

extern "C" {

int bn_gqa_decode_planned(int dtype, const void *q, const void *k_cache, const void *v_cache,
                          const int32_t *seq_lens, const int32_t *h_seq_lens, void *o, int batch,
                          int max_len, int n_heads, int n_kv_heads, int head_dim, float scale,
                          void *workspace, size_t workspace_bytes, void *stream) {
  return gqa_decode_planned_impl(dtype, q, k_cache, v_cache, seq_lens, h_seq_lens, o, batch, max_len,
                                 n_heads, n_kv_heads, head_dim, scale, workspace, workspace_bytes,
                                 stream, nullptr);
}

int bn_gqa_decode_planned_strided(int dtype, const void *q, const void *k_cache,
                                  const void *v_cache, const int32_t *seq_lens,
                                  const int32_t *h_seq_lens, void *o, int batch, int max_len,
                                  int n_heads, int n_kv_heads, int head_dim,
                                  int64_t cache_seq_stride, int64_t cache_head_stride,
                                  int64_t cache_row_stride, float scale, void *workspace,
                                  size_t workspace_bytes, void *stream) {
  const int64_t strides[3] = {cache_seq_stride, cache_head_stride, cache_row_stride};
  return gqa_decode_planned_impl(dtype, q, k_cache, v_cache, seq_lens, h_seq_lens, o, batch, max_len,
                                 n_heads, n_kv_heads, head_dim, scale, workspace, workspace_bytes,
                                 stream, strides);
}

}  // extern "C"
