// bn_fused_head.hip -- the reference's fused-head attention chain in one launch.
//
// Replaces the chain of llama_layers.hpp:83-109 (fp32):
//   K_rep = repeat_kv(K), V_rep = repeat_kv(V)       (:87-89, :131-168)
//   S = Q @ K_rep^T                                    (:96-98, op_mm)
//   S = S * scale                                      (:101, op_multiply)
//   P = softmax(S, causal, seq_offset)                 (:105, op_softmax.cuh:77-151)
//   O = P @ V_rep                                      (:108-109, op_mm)
// Q is [Sq, H*D]; the chain's scores contract over ALL H*D columns, so one
// probability matrix is shared by every head.  With n_rep = H / KV and head
// h reading KV head h / n_rep (:159-163):
//   S[i][j] = sum_g Qsum_g[i] . K_g[j],   Qsum_g[i] = sum_{r < n_rep} Q_{g*n_rep + r}[i]
// a KV*D-wide contraction instead of an H*D-wide one over K_rep, and
//   O[i][h*D + d] = (P @ V_{h / n_rep})[i][d]
// so the n_rep heads of a group receive the same values.  Neither K_rep,
// V_rep nor the Sq x Sk matrices exist here.
//
// Work decomposition: a 256-thread workgroup (4 waves) owns R = 4 query rows
// and walks the visible keys in tiles of 64 with an online softmax:
//   1. the rows' Qsum (R x KV*D) is formed once into LDS;
//   2. scores: thread (wave w, lane l) forms the R partial dots of key l over
//      the w-th quarter of the contraction (each K element is loaded once per
//      workgroup and used R times); the quarters meet in LDS;
//   3. softmax: wave r owns row r (max, exponentials and row sum by wave
//      reductions) and publishes P^T and the rescale factor;
//   4. P.V: thread (w, l) accumulates columns 4l.. of every row over the keys
//      j = w mod 4 of the tile (a wave reads whole V rows: coalesced);
//   5. the four key-split partials meet in LDS and every thread writes its
//      share of the R x H*D output, each group's values to its n_rep heads.
// Why VALU and not fp32 MFMA: at the config this chain runs on (Sq = Sk =
// 128, KV*D = 256) the launch is latency-bound -- 17 MFLOP and 2.4 MB of
// algorithmic traffic, i.e. well under a microsecond at either roofline.
// The v_mfma_f32_16x16x4f32 rate is 2x VALU FMA but needs 16-row tiles:
// 4x fewer workgroups (8 at Sq = 128) and 4x the per-workgroup work, so the
// last workgroup would finish later.  Four rows per workgroup also balance
// the K/V bytes a workgroup pulls from L2 against its FMAs (R FMAs per
// loaded float).  Measured (rocprofv3, 300 launches): 13.0 us at Sq = 128
// (2 key tiles on the longest rows), 34.3 us at 512 (8 tiles): ~6 us fixed
// (launch, Q and the first tile's K/V, output) and ~3.5 us per tile, of
// which the dot products take ~0.9 and P.V ~0.4; the rest is the 128 KB of
// K and V each workgroup pulls per tile through one CU.
#include <algorithm>

#include "bn_common.hpp"

namespace bn {
namespace {

constexpr int kRows = 4;      // query rows per workgroup (= waves)
constexpr int kTile = 64;     // keys per tile (= lanes)
constexpr int kMaxKvd = 512;  // KV*D limit: 2 column chunks of 256
constexpr int kRepChunk = 8;  // Q heads summed per batch of loads

struct FusedHeadParams {
  const float *q, *k, *v;
  float *o;
  int64_t ldq, ldk, ldv, ldo;  // row strides in elements (columns contiguous)
  int sq, sk;
  int n_heads, head_dim, kvd, n_rep;
  float scale;
  int causal, seq_offset;
};

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ float4 zero4() { return float4{0.f, 0.f, 0.f, 0.f}; }

// Max over the wave without an LDS round trip: DPP inside each 16-lane row
// (quad xor 1, quad xor 2, half-row mirror, row mirror: every source lane is
// in the row), then the four row maxima by readlane.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xf, 0xf, false));
}
__device__ __forceinline__ float lane_of(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ __forceinline__ float wave_max_dpp(float x) {
  x = fmaxf(x, dpp_mov<0xB1>(x));
  x = fmaxf(x, dpp_mov<0x4E>(x));
  x = fmaxf(x, dpp_mov<0x141>(x));
  x = fmaxf(x, dpp_mov<0x140>(x));
  return fmaxf(fmaxf(lane_of(x, 0), lane_of(x, 16)), fmaxf(lane_of(x, 32), lane_of(x, 48)));
}

// KC = 256-column chunks of KV*D (1: KV*D <= 256, 2: <= 512).  The launch is
// latency-bound, so every phase issues all of its global loads before the
// first use: K and V of tile 0, then Q (the rows' heads) behind them; with
// KC = 1 the K quarter of tile t+1 is in flight during the softmax and P.V of
// tile t, and its V rows during the softmax of tile t+1.
// FQ: the contraction quarter in float4s when fixed at compile time (16 for
// KV*D = 256: no per-load predicates), 0 when read from p.kvd.
template <int KC, int FQ>
__global__ __launch_bounds__(256) void fused_head_attention_kernel(FusedHeadParams p) {
  constexpr int NQ = 4 * KC;   // float4s of one contraction quarter per 256 columns
  // KC = 1: the next tile's K and V stay in registers across a tile (128
  // VGPRs); KC = 2 would need 256, so it loads K, then V, per tile
  constexpr bool kPipe = KC == 1;
  __shared__ float4 qs[kRows][kMaxKvd / 4];       // Qsum rows
  __shared__ float part[4][kRows][kTile];         // quarter partial dots
  __shared__ float4 pt[kTile];                    // P^T: key -> 4 rows
  __shared__ float alpha_s[kRows], lsum_s[kRows];
  __shared__ float4 obuf[4][kRows][kMaxKvd / 4];  // key-split partial O

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int r0 = blockIdx.x * kRows;
  const int nrows = min(kRows, p.sq - r0);
  const int kvd4 = p.kvd >> 2, D = p.head_dim;
  const int quarter4 = FQ ? FQ : kvd4 >> 2;  // float4s per contraction quarter (<= 4*NQ)

  // visible keys of the block: j < kend (row r also needs j <= r0 + r + off)
  const int last = r0 + nrows - 1;
  int kend = p.sk;
  if (p.causal) kend = (int)min((int64_t)p.sk, max((int64_t)0, (int64_t)last + p.seq_offset + 1));

  // K quarter w of key kb + lane, V rows kb + w + 4u (u < 16) at columns 4*lane + 256*cc
  float4 kx[4 * NQ];
  float4 vx[KC][16];
  auto load_k = [&](int kb) __attribute__((always_inline)) {
    const int j = min(kb + lane, kend - 1);
    const float *kr = p.k + (int64_t)j * p.ldk + 4 * w * quarter4;
#pragma unroll
    for (int i = 0; i < 4 * NQ; ++i) kx[i] = (FQ || i < quarter4) ? ld4(kr + 4 * i) : zero4();
  };
  // Rows past the tile's last key are read at the last key (in bounds, P = 0
  // there): no branch around the loads, so their waits stay counted.
  auto load_v = [&](int kb) __attribute__((always_inline)) {
    const int nk = min(kTile, kend - kb);
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const float *vr = p.v + (int64_t)(kb + min(w + 4 * u, nk - 1)) * p.ldv;
#pragma unroll
      for (int cc = 0; cc < KC; ++cc) {
        const int c = 4 * lane + 256 * cc;
        vx[cc][u] = (FQ || c < p.kvd) ? ld4(vr + c) : zero4();
      }
    }
  };

  // tile 0's K and V go out first; the Q loads queue behind them
  if (kPipe && kend > 0) {
    load_k(0);
    load_v(0);
  }
  // 1. Qsum: column c = g*D + d sums Q columns (g*n_rep + r)*D + d, r ascending
  for (int e = tid; e < kRows * kvd4; e += 256) {
    const int r = e / kvd4, c = 4 * (e - r * kvd4);
    const int g = c / D, d = c - g * D;
    // rows past the last one and heads past the group re-read a valid
    // element and are weighted 0: the loads need no branch
    float4 acc = zero4();
    const float row_w = r < nrows ? 1.f : 0.f;
    const float *src = p.q + (int64_t)(r0 + min(r, nrows - 1)) * p.ldq + (int64_t)g * p.n_rep * D + d;
    for (int rb = 0; rb < p.n_rep; rb += kRepChunk) {
      float4 x[kRepChunk];
#pragma unroll
      for (int rr = 0; rr < kRepChunk; ++rr) x[rr] = ld4(src + min(rb + rr, p.n_rep - 1) * D);
#pragma unroll
      for (int rr = 0; rr < kRepChunk; ++rr) {
        const float f = rb + rr < p.n_rep ? row_w : 0.f;
        acc.x = fmaf(f, x[rr].x, acc.x);
        acc.y = fmaf(f, x[rr].y, acc.y);
        acc.z = fmaf(f, x[rr].z, acc.z);
        acc.w = fmaf(f, x[rr].w, acc.w);
      }
    }
    qs[r][c >> 2] = acc;
  }
  // row w's state (wave w): running max, and this lane's share of the row sum
  // (the lanes' shares meet once, after the last tile)
  float m_row = -INFINITY, l_lane = 0.f;
  float4 oacc[kRows][KC];
#pragma unroll
  for (int r = 0; r < kRows; ++r)
#pragma unroll
    for (int cc = 0; cc < KC; ++cc) oacc[r][cc] = zero4();
  __syncthreads();

  const int64_t row_lim = (int64_t)(r0 + w) + p.seq_offset;  // wave w runs row r0 + w
  for (int kb = 0; kb < kend; kb += kTile) {
    const int nk = min(kTile, kend - kb);
    if (!kPipe) load_k(kb);
    // 2. partial dots of key kb + lane over quarter w
    {
      float acc[kRows] = {0.f, 0.f, 0.f, 0.f};
      const float4 *qq = &qs[0][w * quarter4];
#pragma unroll
      for (int i = 0; i < 4 * NQ; ++i) {
        if (FQ || i < quarter4) {
#pragma unroll
          for (int r = 0; r < kRows; ++r) {
            const float4 a = qq[r * (kMaxKvd / 4) + i];
            acc[r] = fmaf(a.x, kx[i].x, acc[r]);
            acc[r] = fmaf(a.y, kx[i].y, acc[r]);
            acc[r] = fmaf(a.z, kx[i].z, acc[r]);
            acc[r] = fmaf(a.w, kx[i].w, acc[r]);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < kRows; ++r) part[w][r][lane] = acc[r];
    }
    if (kPipe && kb + kTile < kend) load_k(kb + kTile);  // next tile's K in flight
    if (!kPipe) load_v(kb);
    __syncthreads();
    // 3. online softmax of row w over the tile
    {
      const int j = kb + lane;
      float s = ((part[0][w][lane] + part[1][w][lane]) + part[2][w][lane]) + part[3][w][lane];
      s *= p.scale;
      const bool vis = w < nrows && lane < nk && (!p.causal || (int64_t)j <= row_lim);
      s = vis ? s : -INFINITY;
      const float m_new = fmaxf(m_row, wave_max_dpp(s));
      const float mn = m_new == -INFINITY ? 0.f : m_new;
      const float pj = vis ? expf(s - mn) : 0.f;
      const float alpha = expf(m_row - mn);  // m_row = -inf -> 0 (l and O are 0 then)
      l_lane = fmaf(l_lane, alpha, pj);
      m_row = m_new;
      reinterpret_cast<float *>(&pt[lane])[w] = pj;
      if (lane == 0) alpha_s[w] = alpha;
    }
    __syncthreads();
    // 4. O += P V over keys j = w (mod 4) of the tile
    {
      float al[kRows];
#pragma unroll
      for (int r = 0; r < kRows; ++r) al[r] = alpha_s[r];
#pragma unroll
      for (int r = 0; r < kRows; ++r)
#pragma unroll
        for (int cc = 0; cc < KC; ++cc) {
          oacc[r][cc].x *= al[r];
          oacc[r][cc].y *= al[r];
          oacc[r][cc].z *= al[r];
          oacc[r][cc].w *= al[r];
        }
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const float4 pp = pt[w + 4 * u];  // 0 past the tile's last key
        const float pr[kRows] = {pp.x, pp.y, pp.z, pp.w};
#pragma unroll
        for (int cc = 0; cc < KC; ++cc)
#pragma unroll
          for (int r = 0; r < kRows; ++r) {
            oacc[r][cc].x = fmaf(pr[r], vx[cc][u].x, oacc[r][cc].x);
            oacc[r][cc].y = fmaf(pr[r], vx[cc][u].y, oacc[r][cc].y);
            oacc[r][cc].z = fmaf(pr[r], vx[cc][u].z, oacc[r][cc].z);
            oacc[r][cc].w = fmaf(pr[r], vx[cc][u].w, oacc[r][cc].w);
          }
      }
    }
    if (kPipe && kb + kTile < kend) load_v(kb + kTile);
  }

  // 5. merge the key-split partials, normalise, write each group to its heads
#pragma unroll
  for (int r = 0; r < kRows; ++r)
#pragma unroll
    for (int cc = 0; cc < KC; ++cc) {
      const int c = 4 * lane + 256 * cc;
      if (c < p.kvd) obuf[w][r][c >> 2] = oacc[r][cc];
    }
  const float l_row = wave_sum(l_lane);
  if (lane == 0) lsum_s[w] = l_row;
  __syncthreads();
  const int hd4 = (p.n_heads * D) >> 2;
  for (int e = tid; e < nrows * hd4; e += 256) {
    const int r = e / hd4, c = 4 * (e - r * hd4);
    const int h = c / D, d = c - h * D;
    const int src = ((h / p.n_rep) * D + d) >> 2;
    const float4 a = obuf[0][r][src], b = obuf[1][r][src], x = obuf[2][r][src],
                 y = obuf[3][r][src];
    const float l = lsum_s[r];
    float4 out = zero4();
    if (l > 0.f) {  // a row with no visible key: the chain's P row is all 0
      const float inv = 1.f / l;
      out.x = (((a.x + b.x) + x.x) + y.x) * inv;
      out.y = (((a.y + b.y) + x.y) + y.y) * inv;
      out.z = (((a.z + b.z) + x.z) + y.z) * inv;
      out.w = (((a.w + b.w) + x.w) + y.w) * inv;
    }
    *reinterpret_cast<float4 *>(p.o + (int64_t)(r0 + r) * p.ldo + c) = out;
  }
}

// ------------------------------------------------------- matrix-core path
// Longer prompts (seq_q >= kMfmaMinRows) with KV*D = 256 (TinyLLaMA's 4 KV
// heads of 64) run the same chain on v_mfma_f32_32x32x2f32, in three
// launches:
//   1. fh_qsum_kernel: Qs[i][c] = c2 * sum_{r < n_rep} Q_{g*n_rep + r}[i][d]
//      (c = g*D + d, summed in r order; c2 = scale * log2 e, so the scores
//      come out in log2 units), [seq_q, 256] in the workspace.
//   2. fh_mfma_kernel: one workgroup per block of 32 query rows x 128 keys.
//      Wave w forms S^T = K.Qs^T of the block's four 32-key tiles over its
//      quarter (64 columns) of the contraction; the four quarters meet in LDS
//      and are summed in wave order, so every wave holds the same 128 x 32
//      scores.  Each wave masks them, takes the block's row max m, forms
//      P = exp2(s - m) and l = sum P, and O[:, 64w .. 64w+63] = P.V for its
//      quarter of the value columns (P straight from the score registers as
//      the B operand).  The block writes its record (m, l, O[32][256]).
//   3. fh_merge_kernel: each query row merges the records of its row tile
//      (max of m, exp2-weighted sums of l and O), normalises, and writes the
//      values of KV head g to the row's n_rep heads of group g.
// Per block a wave runs 128 MFMAs for S and 128 for P.V; the blocks of a
// prompt spread over every compute unit, where the VALU kernel's longest
// rows walk every key tile on one compute unit each.
constexpr int kMfmaMinRows = 512;  // shorter prompts: the VALU kernel (faster at 256 rows)
constexpr int FH_KVD = 256, FH_ROWS = 32, FH_KEYS = 128;
constexpr int FH_REC = 2 * FH_ROWS + FH_ROWS * FH_KVD;  // m[32], l[32], O[32][256]

typedef float fh_f32x16 __attribute__((ext_vector_type(16)));

struct FhParams {
  const float *q, *k, *v;
  float *o, *qs, *part;
  int64_t ldq, ldk, ldv, ldo;
  int sq, sk, n_heads, head_dim, n_rep, n_kc, causal, seq_offset;
  float c2;  // scale * log2(e)
};

// visible keys of query row `row`: [0, key_end)
__device__ __forceinline__ int fh_key_end(const FhParams &p, int row) {
  if (!p.causal) return p.sk;
  const int64_t e = (int64_t)row + p.seq_offset + 1;
  return (int)(e < 0 ? 0 : (e > p.sk ? p.sk : e));
}

__global__ __launch_bounds__(256) void fh_qsum_kernel(FhParams p) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)p.sq * (FH_KVD / 4)) return;
  const int row = (int)(idx / (FH_KVD / 4)), c = (int)(idx % (FH_KVD / 4)) * 4;
  const int g = c / p.head_dim, d = c - g * p.head_dim;
  const float *qr = p.q + (int64_t)row * p.ldq + (int64_t)g * p.n_rep * p.head_dim + d;
  float4 a = ld4(qr);
  for (int r = 1; r < p.n_rep; ++r) {
    const float4 b = ld4(qr + (int64_t)r * p.head_dim);
    a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
  }
  *reinterpret_cast<float4 *>(p.qs + (int64_t)row * FH_KVD + c) =
      make_float4(a.x * p.c2, a.y * p.c2, a.z * p.c2, a.w * p.c2);
}

__global__ __launch_bounds__(256, 2) void fh_mfma_kernel(FhParams p) {
  // the four waves' partial scores: [wave][key tile][register group][lane]
  __shared__ float4 sbuf[4][4][4][64];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int r32 = lane & 31, hf = lane >> 5;
  const int kc = blockIdx.x % p.n_kc, rt = blockIdx.x / p.n_kc;
  const int row0 = rt * FH_ROWS, key0 = kc * FH_KEYS;
  const int kend_tile = fh_key_end(p, min(row0 + FH_ROWS - 1, p.sq - 1));
  if (key0 >= kend_tile) return;  // no record: the merge counts the blocks the same way

  // B operand of S^T: query row0 + r32, contraction slot (4u + e, hf) =
  // column 64w + 8u + 4hf + e of Qs (rows past seq_q: zeros)
  const int qrow = row0 + r32;
  float qreg[32];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const float4 a = qrow < p.sq ? ld4(p.qs + (int64_t)qrow * FH_KVD + 64 * w + 8 * u + 4 * hf) : zero4();
    qreg[4 * u] = a.x; qreg[4 * u + 1] = a.y; qreg[4 * u + 2] = a.z; qreg[4 * u + 3] = a.w;
  }
  // A operand: key key0 + 32kt + r32 (clamped into the cache; masked below),
  // the same contraction columns
  auto load_k = [&](int kt, float4 (&kr)[8]) __attribute__((always_inline)) {
    const int key = min(key0 + 32 * kt + r32, p.sk - 1);
    const float *kp = p.k + (int64_t)key * p.ldk + 64 * w + 4 * hf;
#pragma unroll
    for (int u = 0; u < 8; ++u) kr[u] = ld4(kp + 8 * u);
  };
  fh_f32x16 s[4];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    float4 cur[8];
    load_k(kt, cur);
    s[kt] = fh_f32x16{};
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      s[kt] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur[u].x, qreg[4 * u], s[kt], 0, 0, 0);
      s[kt] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur[u].y, qreg[4 * u + 1], s[kt], 0, 0, 0);
      s[kt] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur[u].z, qreg[4 * u + 2], s[kt], 0, 0, 0);
      s[kt] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur[u].w, qreg[4 * u + 3], s[kt], 0, 0, 0);
    }
  }
  // the quarters of the contraction meet in LDS, summed in wave order
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      sbuf[w][kt][g][lane] = make_float4(s[kt][4 * g], s[kt][4 * g + 1], s[kt][4 * g + 2], s[kt][4 * g + 3]);
  __syncthreads();
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float4 a = sbuf[0][kt][g][lane];
#pragma unroll
      for (int w2 = 1; w2 < 4; ++w2) {
        const float4 b = sbuf[w2][kt][g][lane];
        a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
      }
      s[kt][4 * g] = a.x; s[kt][4 * g + 1] = a.y; s[kt][4 * g + 2] = a.z; s[kt][4 * g + 3] = a.w;
    }

  // mask, row max, P = exp2(s - m), row sum; register i of s[kt] is key
  // key0 + 32kt + 8(i/4) + 4hf + i%4 of query qrow
  const int kend_row = qrow < p.sq ? fh_key_end(p, qrow) : 0;
  float mx = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = key0 + 32 * kt + 8 * (i >> 2) + 4 * hf + (i & 3);
      const float v = key < kend_row ? s[kt][i] : -INFINITY;
      s[kt][i] = v;
      mx = fmaxf(mx, v);
    }
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  const float mu = mx == -INFINITY ? 0.f : mx;
  float l = 0.f;
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float e = __builtin_amdgcn_exp2f(s[kt][i] - mu);
      s[kt][i] = e;
      l += e;
    }
  l += __shfl_xor(l, 32, 64);

  // O^T[value column][query] += V^T P^T over the block's keys: A = V^T (lane:
  // column slot r32 of tile dt = value column 64w + 2*r32 + dt, key of the
  // step's half hf), B = P^T (the score registers)
  fh_f32x16 o[2] = {fh_f32x16{}, fh_f32x16{}};
  auto load_v = [&](int kt, float2 (&vr)[16]) __attribute__((always_inline)) {
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = min(key0 + 32 * kt + 8 * g + 4 * hf + e, p.sk - 1);
        vr[4 * g + e] = *reinterpret_cast<const float2 *>(p.v + (int64_t)key * p.ldv + 64 * w + 2 * r32);
      }
  };
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    float2 cur[16];
    load_v(kt, cur);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      o[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur[i].x, s[kt][i], o[0], 0, 0, 0);
      o[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur[i].y, s[kt][i], o[1], 0, 0, 0);
    }
  }

  // the block's record: m and l per query (wave 0), O[query][column]:
  // register i of o[dt] is column 64w + 2*(8(i/4) + 4hf + i%4) + dt of query qrow
  float *rec = p.part + (int64_t)blockIdx.x * FH_REC;
  if (w == 0 && hf == 0) {
    rec[r32] = mx;
    rec[FH_ROWS + r32] = l;
  }
  float *orow = rec + 2 * FH_ROWS + r32 * FH_KVD + 64 * w;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int c0 = 2 * (8 * g + 4 * hf);
    *reinterpret_cast<float4 *>(orow + c0) = make_float4(o[0][4 * g], o[1][4 * g], o[0][4 * g + 1], o[1][4 * g + 1]);
    *reinterpret_cast<float4 *>(orow + c0 + 4) =
        make_float4(o[0][4 * g + 2], o[1][4 * g + 2], o[0][4 * g + 3], o[1][4 * g + 3]);
  }
}

__global__ __launch_bounds__(256) void fh_merge_kernel(FhParams p) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)p.sq * (FH_KVD / 4)) return;
  const int row = (int)(idx / (FH_KVD / 4)), c = (int)(idx % (FH_KVD / 4)) * 4;
  const int rt = row / FH_ROWS, r = row % FH_ROWS;
  const int kend_tile = fh_key_end(p, min(rt * FH_ROWS + FH_ROWS - 1, p.sq - 1));
  const int nblk = (kend_tile + FH_KEYS - 1) / FH_KEYS;  // the blocks that wrote a record
  const float *rec0 = p.part + (int64_t)rt * p.n_kc * FH_REC;
  // records four at a time, their loads issued together (slots past nblk
  // read the last record and are skipped by a select)
  float M = -INFINITY;
  for (int b = 0; b < nblk; b += 4) {
    float m4[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) m4[j] = rec0[(int64_t)min(b + j, nblk - 1) * FH_REC + r];
#pragma unroll
    for (int j = 0; j < 4; ++j) M = b + j < nblk ? fmaxf(M, m4[j]) : M;
  }
  float4 out = zero4();
  if (M != -INFINITY) {  // a row with no visible key: the chain's P row is all 0
    float L = 0.f;
    float4 A = zero4();
    for (int b = 0; b < nblk; b += 4) {
      float m4[4], l4[4];
      float4 a4[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float *rec = rec0 + (int64_t)min(b + j, nblk - 1) * FH_REC;
        m4[j] = rec[r];
        l4[j] = rec[FH_ROWS + r];
        a4[j] = ld4(rec + 2 * FH_ROWS + r * FH_KVD + c);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (b + j >= nblk) break;
        const float f = __builtin_amdgcn_exp2f(m4[j] - M);  // a block the row cannot see: 0
        L = fmaf(l4[j], f, L);
        A.x = fmaf(a4[j].x, f, A.x); A.y = fmaf(a4[j].y, f, A.y);
        A.z = fmaf(a4[j].z, f, A.z); A.w = fmaf(a4[j].w, f, A.w);
      }
    }
    const float inv = 1.f / L;
    out = make_float4(A.x * inv, A.y * inv, A.z * inv, A.w * inv);
  }
  // KV head g's values go to the n_rep heads of group g
  const int g = c / p.head_dim, d = c - g * p.head_dim;
  float *orow = p.o + (int64_t)row * p.ldo + (int64_t)g * p.n_rep * p.head_dim + d;
  for (int h = 0; h < p.n_rep; ++h) *reinterpret_cast<float4 *>(orow + (int64_t)h * p.head_dim) = out;
}

// A view the kernel can read with float4 loads: fp32, columns contiguous,
// every row on a 16-byte boundary.
bool vec4_rows(const bn_view *v) { return rows_aligned(v, 16); }

}  // namespace
}  // namespace bn

using namespace bn;

extern "C" int bn_fused_head_attention(const bn_view *q, const bn_view *k, const bn_view *v,
                                       const bn_view *o, int n_heads, int n_kv_heads,
                                       int head_dim, float scale, int causal, int seq_offset,
                                       void *stream) {
  const char *op = "Fused-head attention";
  const unsigned mask = 1u << BN_F32;
  int st;
  if ((st = check_view(q, op, "query", mask))) return st;
  if ((st = check_view(k, op, "key", mask))) return st;
  if ((st = check_view(v, op, "value", mask))) return st;
  if ((st = check_view(o, op, "output", mask))) return st;
  if (n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || n_heads % n_kv_heads != 0)
    return fail(BN_ERR_SHAPE, std::string(op) + ": n_heads must be a positive multiple of n_kv_heads");
  const int64_t hd = (int64_t)n_heads * head_dim, kvd = (int64_t)n_kv_heads * head_dim;
  if (q->w != hd || o->w != hd || o->h != q->h)
    return fail(BN_ERR_SHAPE, std::string(op) + ": query and output must be [seq_q, n_heads*head_dim]");
  if (k->w != kvd || v->w != kvd || v->h != k->h)
    return fail(BN_ERR_SHAPE, std::string(op) + ": key and value must be [seq_kv, n_kv_heads*head_dim]");
  if (head_dim % 4 != 0 || kvd % 16 != 0 || kvd > kMaxKvd)
    return fail(BN_ERR_UNSUPPORTED,
                std::string(op) + ": needs head_dim % 4 == 0, n_kv_heads*head_dim % 16 == 0 and <= " +
                    std::to_string(kMaxKvd) + " (got head_dim " + std::to_string(head_dim) +
                    ", n_kv_heads*head_dim " + std::to_string(kvd) + ")");
  if ((st = require_device(op, {q, k, v, o}))) return st;
  if (!vec4_rows(q) || !vec4_rows(k) || !vec4_rows(v) || !vec4_rows(o))
    return fail(BN_ERR_UNSUPPORTED,
                std::string(op) + ": views need contiguous columns and rows on 16-byte boundaries");
  if ((st = ensure_device())) return st;
  if (q->h == 0) return BN_OK;
  if (kvd == FH_KVD && q->h >= kMfmaMinRows) {  // the matrix-core path
    FhParams f;
    f.q = reinterpret_cast<const float *>(q->data) + q->offset;
    f.k = reinterpret_cast<const float *>(k->data) + k->offset;
    f.v = reinterpret_cast<const float *>(v->data) + v->offset;
    f.o = reinterpret_cast<float *>(o->data) + o->offset;
    f.ldq = q->stride_h; f.ldk = k->stride_h; f.ldv = v->stride_h; f.ldo = o->stride_h;
    f.sq = q->h; f.sk = k->h;
    f.n_heads = n_heads; f.head_dim = head_dim; f.n_rep = n_heads / n_kv_heads;
    f.n_kc = (k->h + FH_KEYS - 1) / FH_KEYS;
    f.causal = causal ? 1 : 0;
    f.seq_offset = seq_offset;
    f.c2 = scale * 1.4426950408889634f;
    const int n_rt = (q->h + FH_ROWS - 1) / FH_ROWS;
    const size_t qs_bytes = (size_t)q->h * FH_KVD * sizeof(float);
    const size_t part_bytes = (size_t)n_rt * std::max(f.n_kc, 1) * FH_REC * sizeof(float);
    void *ws = nullptr;
    if ((st = bn_alloc(&ws, qs_bytes + part_bytes, stream))) return st;
    f.qs = (float *)ws;
    f.part = (float *)((char *)ws + qs_bytes);
    hipStream_t s = as_stream(stream);
    const unsigned nvec = (unsigned)(((int64_t)q->h * (FH_KVD / 4) + 255) / 256);
    hipLaunchKernelGGL(fh_qsum_kernel, dim3(nvec), dim3(256), 0, s, f);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && f.n_kc > 0) {
      hipLaunchKernelGGL(fh_mfma_kernel, dim3((unsigned)(n_rt * f.n_kc)), dim3(256), 0, s, f);
      e = hipGetLastError();
    }
    if (e == hipSuccess) {
      hipLaunchKernelGGL(fh_merge_kernel, dim3(nvec), dim3(256), 0, s, f);
      e = hipGetLastError();
    }
    st = e == hipSuccess ? BN_OK : hip_fail(e, __FILE__, __LINE__);
    const int st2 = bn_free(ws, stream);
    return st ? st : st2;
  }
  FusedHeadParams p;
  p.q = reinterpret_cast<const float *>(q->data) + q->offset;
  p.k = reinterpret_cast<const float *>(k->data) + k->offset;
  p.v = reinterpret_cast<const float *>(v->data) + v->offset;
  p.o = reinterpret_cast<float *>(o->data) + o->offset;
  p.ldq = q->stride_h;
  p.ldk = k->stride_h;
  p.ldv = v->stride_h;
  p.ldo = o->stride_h;
  p.sq = q->h;
  p.sk = k->h;
  p.n_heads = n_heads;
  p.head_dim = head_dim;
  p.kvd = (int)kvd;
  p.n_rep = n_heads / n_kv_heads;
  p.scale = scale;
  p.causal = causal ? 1 : 0;
  p.seq_offset = seq_offset;
  const dim3 grid((q->h + kRows - 1) / kRows);
  if (kvd == 256)
    hipLaunchKernelGGL((fused_head_attention_kernel<1, 16>), grid, dim3(256), 0, as_stream(stream), p);
  else if (kvd < 256)
    hipLaunchKernelGGL((fused_head_attention_kernel<1, 0>), grid, dim3(256), 0, as_stream(stream), p);
  else
    hipLaunchKernelGGL((fused_head_attention_kernel<2, 0>), grid, dim3(256), 0, as_stream(stream), p);
  BN_LAUNCH_CHECK();
  return BN_OK;
}
