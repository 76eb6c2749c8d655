// bn_prefill_bwd.hip -- backward of the causal GQA prefill attention (bf16,
// head_dim 64) on gfx950 MFMA, flash-style: the probabilities are recomputed
// from the forward's row log-sum-exp, never stored.
//
// For query head h and its KV head g = h / (n_heads/n_kv_heads), with
// P = exp(scale*Q_h K_g^T - lse) on the visible keys (the forward's mask),
//   dP = dO_h V_g^T,  dS = P * (dP - D),  D = rowsum(dO_h * O_h)
//   dQ_h = scale * dS K_g,  dK_g = scale * sum_h dS^T Q_h,  dV_g = sum_h P^T dO_h
// which is the backward of the reference chain's primitives (op_mm,
// op_softmax_backward op_softmax.cuh:182-246, the scale, and repeat_kv's sum
// over the G heads of a group, llama_layers.hpp:159-163).
//
// Two kernels, no atomics:
//   * prefill_bwd_dq_kernel: one workgroup per (batch, head, 128 query rows),
//     4 waves x 32 rows; Q and dO rows stay in registers (B operands), K/V
//     blocks of 64 keys are staged in LDS.  Per 32-key tile:
//       S^T = K Q^T, dP^T = V dO^T  (v_mfma_f32_32x32x16_bf16, lane = query)
//       dQ^T += K^T dS^T            (K^T fragments by ds_read_b64_tr_b16)
//     It also writes D (rowsum dO*O) for the second kernel.
//   * prefill_bwd_dkv_kernel: one workgroup per (batch, KV head, 128 keys),
//     4 waves x 32 keys; K and V rows stay in registers, the G query heads'
//     Q/dO tiles of 32 rows are staged in LDS.  Per tile:
//       S = Q K^T, dP = dO V^T        (lane = key)
//       dV^T += dO^T P, dK^T += Q^T dS
#include <type_traits>

#include "bn_common.hpp"

namespace bn {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int HD = 64;
constexpr int P16 = HD + 8;  // LDS row pitch (elements), 144 B: b128 row reads and tr16 reads
constexpr float kLog2e = 1.4426950408889634f;
// Tiles clear of the causal diagonal and of the sequence end skip the mask
// code (wave-uniform test): +25% on config 2.

struct BwdParams {
  const bf16_t *q, *k, *v, *o, *dout;
  const float *lse;  // [batch, n_heads, seq_q], natural log
  float *dvec;       // [batch, n_heads, seq_q]: D = rowsum(dO * O)
  float *part;       // fp32 dK/dV partial sums per head chunk, or null
  bf16_t *dq, *dk, *dv;
  int64_t q_bs, q_rs, kv_bs, kv_rs, o_bs, o_rs;
  int batch, seq_q, seq_kv, n_heads, group, causal, seq_offset;
  int n_kv, hpw, nchunk;  // KV heads; query heads per dK/dV workgroup; group / hpw
  float c, scale;         // c = scale * log2(e)
};

__device__ __forceinline__ bf16x4_t tr16(const bf16_t *lds) {
  const s16x4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4_t *)(__attribute__((address_space(3))) void *)lds);
  return __builtin_bit_cast(bf16x4_t, r);
}

// exponent base of the recomputed probabilities: P = exp2(s*c - lse2);
// +inf (P = 0) for rows that are padding or see no key
__device__ __forceinline__ float lse2_of(float lse, bool valid) {
  return (valid && lse > -INFINITY) ? lse * kLog2e : INFINITY;
}

// 32x16 transposed fragment of a row-major LDS tile (rows = the contraction
// index): slot j of 16-row chunk u is row 16u + (j/4)*8 + 4hf + j%4, the row
// order of the S / S^T MFMA outputs; lanes (mod 32) give the column d.
__device__ __forceinline__ bf16x8_t tfrag(const bf16_t *tile, int u, int dt, int tr_off) {
  const bf16_t *p = tile + 16 * u * P16 + tr_off + 32 * dt;
  const bf16x4_t lo = tr16(p), hi = tr16(p + 8 * P16);
  return bf16x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// store a transposed accumulator pair acc[dt][i] = X^T[d = 32dt + 8(i/4) + 4hf + i%4][row]
// as bf16 X[row][d] * s
__device__ __forceinline__ void store_rowT(bf16_t *rowp, const f32x16_t (&acc)[2], int hf, float s) {
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      const int d0 = dt * 32 + gi * 8 + hf * 4;
      const uint32_t lo = (uint32_t)f32_to_bf16(acc[dt][4 * gi] * s) |
                          ((uint32_t)f32_to_bf16(acc[dt][4 * gi + 1] * s) << 16);
      const uint32_t hi = (uint32_t)f32_to_bf16(acc[dt][4 * gi + 2] * s) |
                          ((uint32_t)f32_to_bf16(acc[dt][4 * gi + 3] * s) << 16);
      *(uint2 *)(rowp + d0) = make_uint2(lo, hi);
    }
}

// ------------------------------------------------------------------ dQ
__global__ __launch_bounds__(256, 2) void prefill_bwd_dq_kernel(BwdParams p) {
  __shared__ __attribute__((aligned(16))) bf16_t Ks[64 * P16];
  __shared__ __attribute__((aligned(16))) bf16_t Vs[64 * P16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31, hf = lane >> 5;
  const int n_mt = (p.seq_q + 127) / 128;
  int mt, b, h;
  {
    // workgroups are dealt to the 8 XCDs in turn: when the (batch, KV head)
    // groups are a multiple of 8, XCD x takes groups x, x + 8, ... (all their
    // query heads and row tiles, heaviest first), so a group's K/V is read
    // from HBM once per launch and then from that XCD's L2
    const int L = blockIdx.x, NG = p.batch * p.n_kv;
    if (NG % 8 == 0) {
      const int x = L & 7, j = L >> 3, per_mt = (NG >> 3) * p.group;
      mt = n_mt - 1 - j / per_mt;
      const int r = j % per_mt, gi = (r / p.group) * 8 + x;
      b = gi / p.n_kv;
      h = (gi % p.n_kv) * p.group + r % p.group;
    } else {
      mt = n_mt - 1 - L / (p.batch * p.n_heads);  // heaviest first
      const int bh = L % (p.batch * p.n_heads);
      b = bh / p.n_heads;
      h = bh % p.n_heads;
    }
  }
  const int g = h / p.group;
  const int q0 = mt * 128 + wave * 32, qrow = q0 + r32;
  const bool row_ok = qrow < p.seq_q;
  const int qr = min(qrow, p.seq_q - 1);

  const bf16_t *Qr = p.q + b * p.q_bs + (int64_t)qr * p.q_rs + (int64_t)h * HD + 8 * hf;
  const bf16_t *Or = p.o + b * p.o_bs + (int64_t)qr * p.o_rs + (int64_t)h * HD + 8 * hf;
  const bf16_t *Dr = p.dout + b * p.o_bs + (int64_t)qr * p.o_rs + (int64_t)h * HD + 8 * hf;
  // lane holds d = 16t + 8hf .. +7 of its query row (B operands)
  bf16x8_t qreg[4], dreg[4];
  float dsum = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    qreg[t] = *(const bf16x8_t *)(Qr + 16 * t);
    dreg[t] = *(const bf16x8_t *)(Dr + 16 * t);
    const bf16x8_t ot = *(const bf16x8_t *)(Or + 16 * t);
#pragma unroll
    for (int j = 0; j < 8; ++j) dsum += (float)dreg[t][j] * (float)ot[j];
    if (!row_ok) {
      qreg[t] = bf16x8_t{};
      dreg[t] = bf16x8_t{};
    }
  }
  dsum += __shfl_xor(dsum, 32, 64);
  const int64_t rix = ((int64_t)b * p.n_heads + h) * p.seq_q + qrow;
  if (row_ok && hf == 0) p.dvec[rix] = dsum;
  const float lse2 = lse2_of(row_ok ? p.lse[rix] : 0.f, row_ok);
  const long qlimit = p.causal ? (long)qrow + p.seq_offset : (long)p.seq_kv;

  // key range of the workgroup and of this wave
  auto key_end = [&](int last_row) {
    if (!p.causal) return p.seq_kv;
    long e = (long)last_row + p.seq_offset + 1;
    e = e < 0 ? 0 : e;
    return e < p.seq_kv ? (int)e : p.seq_kv;
  };
  const int wg_last = min(mt * 128 + 127, p.seq_q - 1);
  const int nblk = (key_end(wg_last) + 63) / 64;
  const int wave_last = min(q0 + 31, p.seq_q - 1);
  const int wave_kend = wave_last < q0 ? 0 : key_end(wave_last);

  const bf16_t *Kg = p.k + b * p.kv_bs + (int64_t)g * HD;
  const bf16_t *Vg = p.v + b * p.kv_bs + (int64_t)g * HD;
  const int crow = tid >> 3, ccol = (tid & 7) * 8;
  u32x4_t kr[2], vr[2];
  auto gload = [&](int blk) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int key = blk * 64 + crow + 32 * i;
      if (key < p.seq_kv) {
        kr[i] = *(const u32x4_t *)(Kg + (int64_t)key * p.kv_rs + ccol);
        vr[i] = *(const u32x4_t *)(Vg + (int64_t)key * p.kv_rs + ccol);
      } else {
        kr[i] = u32x4_t{0u, 0u, 0u, 0u};
        vr[i] = u32x4_t{0u, 0u, 0u, 0u};
      }
    }
  };
  const int tr_off = (4 * hf + ((lane & 15) >> 2)) * P16 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  f32x16_t acc[2] = {f32x16_t{}, f32x16_t{}};

  if (nblk > 0) gload(0);
  for (int blk = 0; blk < nblk; ++blk) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      *(u32x4_t *)(Ks + (crow + 32 * i) * P16 + ccol) = kr[i];
      *(u32x4_t *)(Vs + (crow + 32 * i) * P16 + ccol) = vr[i];
    }
    __syncthreads();
    if (blk + 1 < nblk) gload(blk + 1);
#pragma unroll
    for (int u2 = 0; u2 < 2; ++u2) {
      const int kb = blk * 64 + 32 * u2;
      if (kb >= wave_kend) continue;  // wave-uniform: keys past this wave's range
      const bf16_t *kt = Ks + 32 * u2 * P16, *vt = Vs + 32 * u2 * P16;
      f32x16_t s = f32x16_t{}, dp = f32x16_t{};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const bf16x8_t ka = *(const bf16x8_t *)(kt + r32 * P16 + 16 * t + 8 * hf);
        const bf16x8_t va = *(const bf16x8_t *)(vt + r32 * P16 + 16 * t + 8 * hf);
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qreg[t], s, 0, 0, 0);
        dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, dreg[t], dp, 0, 0, 0);
      }
      // s[i] = S^T[key kb + 8(i/4) + 4hf + i%4][query qrow]
      bf16x8_t dsb[2];
      auto make_ds = [&](auto masked_tag) __attribute__((always_inline)) {
        constexpr bool MASKED = decltype(masked_tag)::value;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = kb + (i >> 2) * 8 + hf * 4 + (i & 3);
          float pr = __builtin_amdgcn_exp2f(fmaf(s[i], p.c, -lse2));
          if (MASKED && (key >= p.seq_kv || (long)key > qlimit)) pr = 0.f;
          dsb[i >> 3][i & 7] = (__bf16)(pr * (dp[i] - dsum));
        }
      };
      // wave-uniform: every key of the sub-tile exists and every row of the
      // wave sees it (padding rows have P = 0 through lse2 = +inf)
      const bool full = kb + 31 < p.seq_kv && (!p.causal || (long)kb + 31 <= (long)q0 + p.seq_offset);
      if (full)
        make_ds(std::false_type{});
      else
        make_ds(std::true_type{});
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
          acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tfrag(kt, u, dt, tr_off), dsb[u], acc[dt],
                                                            0, 0, 0);
    }
  }
  if (row_ok)
    store_rowT(p.dq + b * p.q_bs + (int64_t)qrow * p.q_rs + (int64_t)h * HD, acc, hf, p.scale);
}

// ----------------------------------------------------------------- dK, dV
// 32-row query tiles staged per barrier (two measured 2% slower)
constexpr int TPI = 1;

// One workgroup per (key block of 128, batch, KV head, head chunk): the
// chunk's hpw query heads are walked together, tile by tile.  With one chunk (hpw = group)
// dK/dV are final and stored as bf16; otherwise each chunk writes its fp32
// partial sums to part [batch][n_kv][nchunk][2][seq_kv][64] and
// prefill_bwd_reduce_kernel adds them up.
__global__ __launch_bounds__(256, 2) void prefill_bwd_dkv_kernel(BwdParams p) {
  __shared__ __attribute__((aligned(16))) bf16_t Qs[2][TPI][32 * P16];
  __shared__ __attribute__((aligned(16))) bf16_t Ds[2][TPI][32 * P16];
  __shared__ __attribute__((aligned(16))) float lse_s[2][TPI][32];
  __shared__ __attribute__((aligned(16))) float dv_s[2][TPI][32];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31, hf = lane >> 5;
  // key block outermost: low block ids (the most query rows under a causal
  // mask) are dispatched first; chunk next, (batch, KV head) innermost, so
  // that when batch*n_kv is a multiple of 8 one XCD holds every chunk of a
  // (batch, KV head) and reads its K/V once
  const int per_bg = p.batch * p.n_kv, per_blk = per_bg * p.nchunk;
  const int kt_blk = (int)(blockIdx.x / per_blk);
  const int rest = (int)(blockIdx.x % per_blk);
  const int bg = rest % per_bg, c = rest / per_bg;
  const int b = bg / p.n_kv, g = bg % p.n_kv;
  const int k0 = kt_blk * 128 + wave * 32, key = k0 + r32;
  const bool key_ok = key < p.seq_kv;
  const int kr_ = min(key, p.seq_kv - 1);

  // K and V rows of this lane's key (B operands), d = 16t + 8hf .. +7
  const bf16_t *Kr = p.k + b * p.kv_bs + (int64_t)kr_ * p.kv_rs + (int64_t)g * HD + 8 * hf;
  const bf16_t *Vr = p.v + b * p.kv_bs + (int64_t)kr_ * p.kv_rs + (int64_t)g * HD + 8 * hf;
  bf16x8_t kreg[4], vreg[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    kreg[t] = key_ok ? *(const bf16x8_t *)(Kr + 16 * t) : bf16x8_t{};
    vreg[t] = key_ok ? *(const bf16x8_t *)(Vr + 16 * t) : bf16x8_t{};
  }

  // query rows that see any key of the block: q + off >= first key
  int q_first = p.causal ? kt_blk * 128 - p.seq_offset : 0;
  q_first = q_first < 0 ? 0 : q_first;
  const int qt0 = q_first / 32, nqt = (p.seq_q + 31) / 32;
  const int per_head = nqt > qt0 ? nqt - qt0 : 0;
  const int ntile = per_head * p.hpw;
  const int h_first = p.group * g + c * p.hpw;
  // tile n: query tile nqt-1 - n/hpw of head h_first + n%hpw.  Row tiles
  // walk down from the last one, every head of the chunk at each, so the
  // resident key blocks of a (batch, KV head) start on the same Q/dO tiles
  // and share them through L2 (config 2: dK/dV reads 155 -> 130 MB, with
  // the order above)

  // staging: per tile, one 16-byte chunk of Q and of dO per thread
  const int crow = tid >> 3, ccol = (tid & 7) * 8;
  u32x4_t qv[TPI], dvv[TPI];
  float lse_r[TPI], dv_r[TPI];
  auto gload = [&](int it) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < TPI; ++t) {
      const int n = it * TPI + t;
      const bool tile_ok = n < ntile;
      const int hh = h_first + (tile_ok ? n % p.hpw : 0);
      const int qt = tile_ok ? nqt - 1 - n / p.hpw : qt0;
      const int qrow = qt * 32 + crow;
      if (tile_ok && qrow < p.seq_q) {
        qv[t] = *(const u32x4_t *)(p.q + b * p.q_bs + (int64_t)qrow * p.q_rs + (int64_t)hh * HD + ccol);
        dvv[t] = *(const u32x4_t *)(p.dout + b * p.o_bs + (int64_t)qrow * p.o_rs + (int64_t)hh * HD + ccol);
      } else {
        qv[t] = u32x4_t{0u, 0u, 0u, 0u};
        dvv[t] = u32x4_t{0u, 0u, 0u, 0u};
      }
      if (tid < 32) {
        const int qq = qt * 32 + tid;
        const bool ok = tile_ok && qq < p.seq_q;
        const int64_t rix = ((int64_t)b * p.n_heads + hh) * p.seq_q + (ok ? qq : 0);
        lse_r[t] = lse2_of(ok ? p.lse[rix] : 0.f, ok);
        dv_r[t] = ok ? p.dvec[rix] : 0.f;
      }
    }
  };
  const int tr_off = (4 * hf + ((lane & 15) >> 2)) * P16 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  f32x16_t dk[2] = {f32x16_t{}, f32x16_t{}}, dv[2] = {f32x16_t{}, f32x16_t{}};

  const int niter = (ntile + TPI - 1) / TPI;
  if (niter > 0) gload(0);
  for (int it = 0; it < niter; ++it) {
    const int buf = it & 1;
#pragma unroll
    for (int t = 0; t < TPI; ++t) {
      *(u32x4_t *)(Qs[buf][t] + crow * P16 + ccol) = qv[t];
      *(u32x4_t *)(Ds[buf][t] + crow * P16 + ccol) = dvv[t];
      if (tid < 32) {
        lse_s[buf][t][tid] = lse_r[t];
        dv_s[buf][t][tid] = dv_r[t];
      }
    }
    __syncthreads();  // also: every wave finished iteration it-2, the last user of buf
    if (it + 1 < niter) gload(it + 1);
#pragma unroll
    for (int t = 0; t < TPI; ++t) {
      const int n = it * TPI + t;
      if (n >= ntile) break;
      const int qb = (nqt - 1 - n / p.hpw) * 32;
      // wave-uniform skip: no query of the tile sees this wave's first key
      if (p.causal && (long)qb + 31 + p.seq_offset < (long)k0) continue;
      const bf16_t *qs = Qs[buf][t], *ds = Ds[buf][t];
      f32x16_t s = f32x16_t{}, dp = f32x16_t{};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bf16x8_t qa = *(const bf16x8_t *)(qs + r32 * P16 + 16 * u + 8 * hf);
        const bf16x8_t da = *(const bf16x8_t *)(ds + r32 * P16 + 16 * u + 8 * hf);
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa, kreg[u], s, 0, 0, 0);
        dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(da, vreg[u], dp, 0, 0, 0);
      }
      // s[i] = S[query qb + 8(i/4) + 4hf + i%4][key]
      bf16x8_t pb[2], sb[2];
      auto make_p = [&](auto masked_tag) __attribute__((always_inline)) {
        constexpr bool MASKED = decltype(masked_tag)::value;
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const float4 l4 = *(const float4 *)(&lse_s[buf][t][8 * gi + 4 * hf]);
          const float4 d4 = *(const float4 *)(&dv_s[buf][t][8 * gi + 4 * hf]);
          const float lv[4] = {l4.x, l4.y, l4.z, l4.w}, dvl[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int i = 4 * gi + e;
            const int qrow = qb + 8 * gi + 4 * hf + e;
            float pr = __builtin_amdgcn_exp2f(fmaf(s[i], p.c, -lv[e]));
            if (MASKED && (!key_ok || (p.causal && (long)key > (long)qrow + p.seq_offset))) pr = 0.f;
            pb[i >> 3][i & 7] = (__bf16)pr;
            sb[i >> 3][i & 7] = (__bf16)(pr * (dp[i] - dvl[e]));
          }
        }
      };
      // wave-uniform: the wave's 32 keys exist and the tile's first row sees
      // all of them (padding rows have P = 0 through lse2 = +inf)
      const bool full = k0 + 31 < p.seq_kv && (!p.causal || (long)qb + p.seq_offset >= (long)k0 + 31);
      if (full)
        make_p(std::false_type{});
      else
        make_p(std::true_type{});
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
          dv[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tfrag(ds, u, dt, tr_off), pb[u], dv[dt], 0, 0, 0);
          dk[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tfrag(qs, u, dt, tr_off), sb[u], dk[dt], 0, 0, 0);
        }
    }
  }
  if (!key_ok) return;
  if (p.part) {
    float *pk = p.part + ((((int64_t)b * p.n_kv + g) * p.nchunk + c) * 2 * p.seq_kv + key) * HD;
    float *pv = pk + (int64_t)p.seq_kv * HD;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        const int d0 = dt * 32 + gi * 8 + hf * 4;
        *(float4 *)(pk + d0) = make_float4(dk[dt][4 * gi], dk[dt][4 * gi + 1], dk[dt][4 * gi + 2], dk[dt][4 * gi + 3]);
        *(float4 *)(pv + d0) = make_float4(dv[dt][4 * gi], dv[dt][4 * gi + 1], dv[dt][4 * gi + 2], dv[dt][4 * gi + 3]);
      }
  } else {
    const int64_t off = b * p.kv_bs + (int64_t)key * p.kv_rs + (int64_t)g * HD;
    store_rowT(p.dk + off, dk, hf, p.scale);
    store_rowT(p.dv + off, dv, hf, 1.f);
  }
}

// dK/dV from the chunks' fp32 partial sums: one thread per 8 consecutive d of
// one (batch, KV head, K-or-V, key) row; reads are contiguous along d and keys
__global__ __launch_bounds__(256) void prefill_bwd_reduce_kernel(BwdParams p, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int dc = (int)(i & 7);
  int64_t r = i >> 3;
  const int key = (int)(r % p.seq_kv);
  r /= p.seq_kv;
  const int which = (int)(r & 1);
  r >>= 1;
  const int g = (int)(r % p.n_kv), b = (int)(r / p.n_kv);
  const int64_t cstride = (int64_t)2 * p.seq_kv * HD;
  const float *src = p.part + ((((int64_t)b * p.n_kv + g) * p.nchunk * 2 + which) * p.seq_kv + key) * HD + 8 * dc;
  float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int c = 0; c < p.nchunk; ++c) {
    const float4 x = *(const float4 *)(src + c * cstride);
    const float4 y = *(const float4 *)(src + c * cstride + 4);
    a[0] += x.x; a[1] += x.y; a[2] += x.z; a[3] += x.w;
    a[4] += y.x; a[5] += y.y; a[6] += y.z; a[7] += y.w;
  }
  const float sc = which ? 1.f : p.scale;
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    w[j] = (uint32_t)f32_to_bf16(a[2 * j] * sc) | ((uint32_t)f32_to_bf16(a[2 * j + 1] * sc) << 16);
  bf16_t *dst = (which ? p.dv : p.dk) + b * p.kv_bs + (int64_t)key * p.kv_rs + (int64_t)g * HD + 8 * dc;
  *(uint4 *)dst = make_uint4(w[0], w[1], w[2], w[3]);
}

// Query heads per dK/dV workgroup: walking the divisors of the group size
// downward, the first that gives enough workgroups (2048 under a causal mask,
// whose key blocks differ in work, else 512), stopping early where the fp32
// partial sums would pass 0.5 byte per 1000 flops of the backward (their
// write and the reduction's read then cost more than the parallelism gains).
// Measured on config 2 (B=4, S=2048, 32/4 heads), TFLOP/s: causal hpw 8/4/2/1
// -> -/392/509/470, non-causal hpw 4/2/1 -> 564/548/523; B=1, S=16384
// causal hpw 4/2/1 -> 551/591/604.
int heads_per_wg(int batch, int seq_q, int seq_kv, int n_heads, int n_kv_heads, int causal) {
  const int group = n_heads / n_kv_heads;
  const int64_t base = (int64_t)batch * n_kv_heads * ((seq_kv + 127) / 128);
  const int64_t min_wg = causal ? 2048 : 512;
  // backward flops / 1000: 5 products of B*H*Sq*Skv*64 MACs (half under a causal mask)
  const double kflops = 10.0 * batch * n_heads * (double)seq_q * seq_kv * HD / (causal ? 2 : 1) / 1000;
  int best = group;
  for (int hpw = group; hpw >= 1; --hpw) {
    if (group % hpw) continue;
    const double part = (hpw < group) ? 2.0 * batch * n_heads / hpw * (double)seq_kv * HD * 4 : 0;
    if (part > 0.5 * kflops) break;
    best = hpw;
    if (base * (group / hpw) >= min_wg) break;
  }
  return best;
}

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

bool aligned16(const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace
}  // namespace bn

using namespace bn;

// D (fp32 [batch, n_heads, seq_q]) and, when the KV heads' query heads are
// split over workgroups, the fp32 dK/dV partial sums
static void workspace_parts(int batch, int seq_q, int seq_kv, int n_heads, int n_kv_heads,
                            int causal, size_t *d_bytes, size_t *part_bytes, int *hpw) {
  *d_bytes = seq_q > 0 ? align256((size_t)batch * n_heads * seq_q * sizeof(float)) : 0;
  *hpw = heads_per_wg(batch, seq_q, seq_kv, n_heads, n_kv_heads, causal);
  const int nchunk = (n_heads / n_kv_heads) / *hpw;
  *part_bytes = (nchunk > 1 && seq_kv > 0)
                    ? (size_t)batch * n_kv_heads * nchunk * 2 * seq_kv * HD * sizeof(float)
                    : 0;
}

extern "C" size_t bn_gqa_prefill_backward_workspace_size(int batch, int seq_q, int seq_kv,
                                                          int n_heads, int n_kv_heads,
                                                          int head_dim, int causal) {
  if (batch <= 0 || seq_q < 0 || seq_kv < 0 || n_heads <= 0 || n_kv_heads <= 0 ||
      n_heads % n_kv_heads != 0 || head_dim != HD)
    return 0;
  size_t d, part;
  int hpw;
  workspace_parts(batch, seq_q, seq_kv, n_heads, n_kv_heads, causal ? 1 : 0, &d, &part, &hpw);
  return d + part;
}

extern "C" int bn_gqa_prefill_backward(
    int dtype, const void *q, const void *k, const void *v, const void *o, const void *dout,
    const float *lse, void *dq, void *dk, void *dv, int batch, int seq_q, int seq_kv, int n_heads,
    int n_kv_heads, int head_dim, int64_t q_batch_stride, int64_t q_row_stride,
    int64_t kv_batch_stride, int64_t kv_row_stride, int64_t o_batch_stride, int64_t o_row_stride,
    float scale, int causal, int seq_offset, void *workspace, size_t workspace_bytes,
    void *stream) {
  const char *op = "GQA prefill backward";
  if (dtype != BN_BF16) return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": dtype must be BF16");
  if (batch < 0 || seq_q < 0 || seq_kv < 0)
    return fail(BN_ERR_SHAPE, std::string(op) + ": negative batch or sequence length");
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0)
    return fail(BN_ERR_SHAPE, std::string(op) + ": num_heads must be a positive multiple of num_kv_heads");
  if (head_dim != HD) return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": head_dim must be 64");
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(BN_ERR_INVALID_ARG, std::string(op) + ": scale must be positive and finite");
  if (batch == 0 || (seq_q == 0 && seq_kv == 0)) return BN_OK;
  if ((seq_q > 0 && (!q || !o || !dout || !lse || !dq)) || (seq_kv > 0 && (!k || !v || !dk || !dv)))
    return fail(BN_ERR_INVALID_ARG, std::string(op) + ": NULL tensor pointer");
  if (q_row_stride < (int64_t)n_heads * HD || o_row_stride < (int64_t)n_heads * HD ||
      kv_row_stride < (int64_t)n_kv_heads * HD)
    return fail(BN_ERR_SHAPE, std::string(op) + ": row stride smaller than heads*head_dim");
  if (batch > 1 && (q_batch_stride < (int64_t)seq_q * q_row_stride ||
                    o_batch_stride < (int64_t)seq_q * o_row_stride ||
                    kv_batch_stride < (int64_t)seq_kv * kv_row_stride))
    return fail(BN_ERR_SHAPE, std::string(op) + ": batch stride smaller than seq*row_stride");
  if ((seq_q > 0 && (!aligned16(q) || !aligned16(o) || !aligned16(dout) || !aligned16(dq))) ||
      (seq_kv > 0 && (!aligned16(k) || !aligned16(v) || !aligned16(dk) || !aligned16(dv))) ||
      (reinterpret_cast<uintptr_t>(lse) & 3u) || q_row_stride % 8 || kv_row_stride % 8 ||
      o_row_stride % 8 || q_batch_stride % 8 || kv_batch_stride % 8 || o_batch_stride % 8)
    return fail(BN_ERR_UNSUPPORTED,
                std::string(op) + ": pointers must be 16-byte aligned and strides multiples of 16 bytes");
  size_t d_bytes, part_bytes;
  int hpw;
  workspace_parts(batch, seq_q, seq_kv, n_heads, n_kv_heads, causal ? 1 : 0, &d_bytes, &part_bytes,
                  &hpw);
  const size_t need = d_bytes + part_bytes;
  if (workspace && workspace_bytes < need)
    return fail(BN_ERR_INVALID_ARG, std::string(op) + ": workspace of " +
                                        std::to_string(workspace_bytes) + " bytes, need " +
                                        std::to_string(need));
  if (workspace && !aligned16(workspace))
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": workspace must be 16-byte aligned");
  const int nchunk = (n_heads / n_kv_heads) / hpw;
  const int64_t n_dq = (int64_t)batch * n_heads * ((seq_q + 127) / 128);
  const int64_t n_dkv = (int64_t)batch * n_kv_heads * nchunk * ((seq_kv + 127) / 128);
  const int64_t n_red = part_bytes ? (int64_t)batch * n_kv_heads * 2 * seq_kv * 8 : 0;
  if (n_dq > 0x7fffffff || n_dkv > 0x7fffffff || (n_red + 255) / 256 > 0x7fffffff)
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": problem too large");
  int st = ensure_device();
  if (st) return st;
  hipStream_t s = as_stream(stream);
  void *ws = workspace;
  bool own = false;
  if (!ws && need) {
    if ((st = bn_alloc(&ws, need, stream))) return st;
    own = true;
  }
  BwdParams p;
  p.q = (const bf16_t *)q; p.k = (const bf16_t *)k; p.v = (const bf16_t *)v;
  p.o = (const bf16_t *)o; p.dout = (const bf16_t *)dout; p.lse = lse;
  p.dvec = (float *)ws;
  p.part = part_bytes ? (float *)((char *)ws + d_bytes) : nullptr;
  p.dq = (bf16_t *)dq; p.dk = (bf16_t *)dk; p.dv = (bf16_t *)dv;
  p.q_bs = q_batch_stride; p.q_rs = q_row_stride; p.kv_bs = kv_batch_stride;
  p.kv_rs = kv_row_stride; p.o_bs = o_batch_stride; p.o_rs = o_row_stride;
  p.batch = batch; p.seq_q = seq_q; p.seq_kv = seq_kv; p.n_heads = n_heads;
  p.group = n_heads / n_kv_heads; p.causal = causal ? 1 : 0; p.seq_offset = seq_offset;
  p.n_kv = n_kv_heads; p.hpw = hpw; p.nchunk = nchunk;
  p.scale = scale; p.c = scale * kLog2e;
  hipError_t e = hipSuccess;
  if (n_dq > 0) {
    hipLaunchKernelGGL(prefill_bwd_dq_kernel, dim3((unsigned)n_dq), dim3(256), 0, s, p);
    e = hipGetLastError();
  }
  if (e == hipSuccess && n_dkv > 0) {
    hipLaunchKernelGGL(prefill_bwd_dkv_kernel, dim3((unsigned)n_dkv), dim3(256), 0, s, p);
    e = hipGetLastError();
  }
  if (e == hipSuccess && n_red > 0) {
    hipLaunchKernelGGL(prefill_bwd_reduce_kernel, dim3((unsigned)((n_red + 255) / 256)), dim3(256),
                       0, s, p, n_red);
    e = hipGetLastError();
  }
  st = e == hipSuccess ? BN_OK : hip_fail(e, __FILE__, __LINE__);
  if (own) {
    const int st2 = bn_free(ws, stream);
    if (st == BN_OK) st = st2;
  }
  return st;
}
