// bn_prefill.hip -- causal GQA prefill attention on gfx950 MFMA.
//
// Replaces, per query head h and its KV head g = h / (n_heads/n_kv_heads),
// the reference chain  Q_h K_g^T -> *scale -> causal softmax(seq_offset) ->
// @ V_g  (llama_layers.py:174-183, llama_layers.hpp:96-109, with the
// repeat_kv mapping of llama_layers.hpp:159-163 done by indexing instead of
// copying) with one flash-style kernel: O(S) memory, K/V blocks staged
// through LDS, online softmax in fp32.
//
// Work decomposition: a 256-thread workgroup (4 waves) owns 4 x 32*RT query
// rows of one (batch, head); each wave owns 32*RT rows (fp32: RT = 1; bf16:
// RT = 2 for long sequences, 1 otherwise).  Key blocks of 64 are staged in
// LDS with the next blocks' global loads in flight while the current block
// is computed.
//
// Per wave and key tile the score tile is computed transposed,
//   S^T[key][query] = K[key][:] . Q[query][:]      (v_mfma_f32_32x32x16_bf16 /
//                                                   v_mfma_f32_32x32x2f32)
// so that each lane holds 16 keys of ONE query: the softmax row max and row
// sum are in-lane plus a single exchange between the two half-waves.  The
// output is accumulated transposed as well,
//   O^T[d][query] += V^T[d][key] . P^T[key][query],
// whose B operand is exactly the P^T registers the softmax produced (no
// shuffles), and whose per-query rescale is a per-lane scalar.
//
// Causal work is unbalanced (row tile m needs m+1 key blocks); workgroups are
// issued heaviest-first.  Only diagonal / tail tiles evaluate the mask.
// Mask: key j is visible to query row i iff j <= i + seq_offset
// (op_softmax.cuh:89-99) and j < seq_kv.
#include "bn_common.hpp"

#include <type_traits>

namespace bn {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int BM = 128;  // query rows per workgroup
constexpr int BN = 64;   // keys per LDS block
constexpr int HD = 64;   // head_dim

struct PrefillParams {
  const void *q, *k, *v;
  void *o;
  int64_t q_bs, q_rs, kv_bs, kv_rs, o_bs, o_rs;
  int batch, seq_q, seq_kv, n_heads, group, n_mt;
  int causal, seq_offset;
  float c;  // scale * log2(e): softmax evaluated as exp2(s*c - m*c)
  float *lse;  // optional [batch, n_heads, seq_q]: natural-log row log-sum-exp of scale*s
};

// natural-log log-sum-exp of the row from its reference max times c (mc)
// and the sum of exp2(s*c - mc): log(sum exp(scale*s)) = (mc + log2(l)) *
// ln 2; -inf when no key is visible
__device__ __forceinline__ float row_lse(float mc, float l) {
  return l > 0.f ? (mc + __log2f(l)) * 0.6931471805599453f : -INFINITY;
}

struct Work {
  int b, h, g, mt;
};

__device__ __forceinline__ Work decode_work(const PrefillParams &p) {
  const int per_m = p.batch * p.n_heads;
  const int L = blockIdx.x;
  Work w;
  w.mt = p.n_mt - 1 - L / per_m;  // heaviest (last) row tiles first
  const int rem = L - (L / per_m) * per_m;
  w.b = rem / p.n_heads;
  w.h = rem - w.b * p.n_heads;
  w.g = w.h / p.group;
  return w;
}

// Key range [0, kend) a set of rows [.., last_row] may see.
__device__ __forceinline__ int key_end(const PrefillParams &p, int last_row) {
  if (!p.causal) return p.seq_kv;
  long e = (long)last_row + p.seq_offset + 1;
  if (e < 0) e = 0;
  return e < p.seq_kv ? (int)e : p.seq_kv;
}

// Online-softmax update of one 64-key block for this lane's query.
// s[kt][i] holds key kb + kt*32 + (i/4)*8 + hf*4 + (i%4).
__device__ __forceinline__ void softmax_block(f32x16_t (&s)[2], float &m, float &l,
                                              f32x16_t (&o)[2], float c, bool need_mask,
                                              int kb, int hf, long qlimit, int seq_kv) {
  if (need_mask) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kb + kt * 32 + (i >> 2) * 8 + hf * 4 + (i & 3);
        if (key >= seq_kv || (long)key > qlimit) s[kt][i] = -INFINITY;
      }
  }
  float mx = s[0][0];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[kt][i]);
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  const float m_new = fmaxf(m, mx);
  const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
  const float mc = m_use * c;
  const float alpha = __builtin_amdgcn_exp2f(m * c - mc);  // m = -inf -> 0
  float rs = 0.f;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float e = __builtin_amdgcn_exp2f(fmaf(s[kt][i], c, -mc));
      s[kt][i] = e;
      rs += e;
    }
  l = l * alpha + rs;  // per half-wave partial; halves are summed at the end
  m = m_new;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
}

// ------------------------------------------------------------------ bf16
// K and V blocks are staged row-major in a double-buffered LDS ring (one
// barrier per block).  K fragments (A of S^T) are ds_read_b128 of K rows; V^T
// fragments (A of O^T) come from the gfx950 transpose read ds_read_b64_tr_b16:
// within each 16-lane group, output lane i slot j is element i%4 of the 8 bytes
// at the address local lane 4j + i/4 supplied, so lanes point at 4 consecutive
// d of one key row and receive one d for 4 consecutive keys.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
constexpr int KP16 = HD + 8;   // K row pitch: 144 B, conflict-free b128 fragment reads
constexpr int VP16 = HD + 32;  // V row pitch: 192 B, transpose reads of 8 rows x 64 B in 2 passes
constexpr int KBUF = BN * KP16, VBUF = BN * VP16;
constexpr float kRescaleLog2 = 8.f;
  // keep a stale row max until the true one is 2^8 larger

__device__ __forceinline__ bf16x4_t tr16(const bf16_t *lds) {
  const s16x4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4_t *)(__attribute__((address_space(3))) void *)lds);
  return __builtin_bit_cast(bf16x4_t, r);
}

// XCD-aware order: consecutive workgroup ids go round-robin to the 8 XCDs
// (each with its own L2); all G query heads of a (batch, KV head) group and
// all its row tiles are placed on one XCD so the group's K/V stays in that
// L2.  Heaviest row tiles first inside each XCD's queue.
__device__ __forceinline__ Work decode_work_xcd(const PrefillParams &p) {
  const int n_kv = p.n_heads / p.group;
  const int NG = p.batch * n_kv;
  if (NG % 8 != 0) return decode_work(p);
  const int L = blockIdx.x, x = L & 7, j = L >> 3;
  const int per_mt = (NG >> 3) * p.group;
  Work w;
  w.mt = p.n_mt - 1 - j / per_mt;
  const int r = j % per_mt;
  const int gi = (r / p.group) * 8 + x;
  w.b = gi / n_kv;
  w.g = gi % n_kv;
  w.h = w.g * p.group + r % p.group;
  return w;
}

// Head-packed work items (bf16, group = 4*RT): one workgroup per (batch, KV
// head, 32 query rows) covering all the group's query heads, wave w on heads
// RT*w .. RT*w + RT-1 of the group.  Every wave then sees the same causal key
// range -- no wave idles in the diagonal blocks -- and only the last 32-key
// tile of the range needs a mask.  Row tiles heaviest first; the workgroups of
// one (batch, KV head) share an XCD when batch*n_kv is a multiple of 8.
__device__ __forceinline__ Work decode_work_packed(const PrefillParams &p) {
  const int n_kv = p.n_heads / p.group;
  const int NG = p.batch * n_kv;
  const int L = blockIdx.x;
  Work w;
  int gi;
  if (NG % 8 == 0) {
    const int x = L & 7, j = L >> 3, per_mt = NG >> 3;
    w.mt = p.n_mt - 1 - j / per_mt;
    gi = (j % per_mt) * 8 + x;
  } else {
    w.mt = p.n_mt - 1 - L / NG;
    gi = L % NG;
  }
  w.b = gi / n_kv;
  w.g = gi % n_kv;
  w.h = w.g * p.group;  // first head of the group
  return w;
}

// Kernel structure -- the softmax does little VALU work per score and runs
// while the matrix cores work:
//   * the fast path is p = exp2(s * c - m * c), c = scale*log2(e), against a
//     reference max m that is NOT recomputed per tile: one fma, one
//     transcendental and half a bf16 pack per score; the tile's row sums run
//     on the matrix cores (v_mfma_f32_16x16x32_bf16 against a 0/1 selector),
//     checked at the start of the next step, when those MFMAs have long
//     finished (measured against a v_dot2 chain on the VALU: +3.5% on
//     config 2, +2.5% on config 5);
//   * m moves only in a rare exact fixup, taken when a tile's row sum exceeds
//     2^16 (some p > 2^16, which includes inf and NaN), and then only when it
//     grew by more than 2^8; the first tile (m = -inf) runs the fixup alone;
//   * software pipeline over 32-key tiles: step t issues O += V_{t-1}^T P_{t-1}
//     and the scores of tile t+1 on the matrix cores, interleaved with the
//     softmax of tile t on the VALU -- three independent pieces of work in
//     one basic block.  Every wave runs the same steps (tiles past its causal
//     range are all -inf, P = 0), so no branch separates them;
//   * K/V blocks are staged with buffer loads whose descriptor starts at the
//     block: the per-thread offset is fixed and rows past seq_kv read as 0.
// LDS: 2-deep K and V rings of 64-key blocks.  Block iteration j runs steps
// 2j+1 and 2j+2, which read only V_j and K_{j+1}; it stores K_{j+2} and
// V_{j+1} (register-staged one iteration earlier) into the buffers of K_j and
// V_{j-1}, last read in iteration j-1 (K_0: in step 0): one barrier per block
// orders them.
constexpr float kSumLimit = 65536.f;
constexpr int kOcc = 2;  // workgroups per CU the register budget is sized for
// step interleave: VALU instructions ahead of the first MFMA, then after each
// MFMA (4 after each of the 20 MFMAs of a step with the row sums on the
// matrix cores; 2 or 6 ahead, and 5 after the 16 products with 2 after the
// row sums, measured equal or slower on configs 2 and 5)
constexpr int kSchedV0 = 4, kSchedV1 = 4;

template <int RT, int OCC, bool HP>
__global__ __launch_bounds__(256, OCC) void prefill_bf16_kernel(PrefillParams p) {
  __shared__ __attribute__((aligned(16))) bf16_t smem[2 * KBUF + 2 * VBUF];
  bf16_t *const kring = smem;
  bf16_t *const vring = smem + 2 * KBUF;
  // rows per wave / per workgroup of one head; head-packed: 32 rows of RT heads
  constexpr int WROWS = HP ? 32 : 32 * RT, WGROWS = HP ? 32 : 4 * WROWS;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31, hf = lane >> 5;
  const Work w = HP ? decode_work_packed(p) : decode_work_xcd(p);
  const bf16_t *Q = (const bf16_t *)p.q + w.b * p.q_bs + (int64_t)w.h * HD;
  const bf16_t *K = (const bf16_t *)p.k + w.b * p.kv_bs + (int64_t)w.g * HD;
  const bf16_t *V = (const bf16_t *)p.v + w.b * p.kv_bs + (int64_t)w.g * HD;
  bf16_t *O = (bf16_t *)p.o + w.b * p.o_bs + (int64_t)w.h * HD;
  const float c = p.c;

  const int q_wave0 = w.mt * WGROWS + (HP ? 0 : wave * WROWS);
  // row tile rt: rows q_wave0 + row_step*rt .., head w.h + head_of(rt)
  constexpr int row_step = HP ? 0 : 32;
  auto head_of = [&](int rt) { return HP ? RT * wave + rt : 0; };

  // Q^T operands: lane holds Q[row][16t + 8hf .. +7], t = 0..3
  bf16x8_t qreg[RT][4];
  int qlimit[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int qrow = q_wave0 + row_step * rt + r32;
    const bf16_t *qp = Q + (int64_t)head_of(rt) * HD + (int64_t)min(qrow, p.seq_q - 1) * p.q_rs + 8 * hf;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      qreg[rt][t] = *(const bf16x8_t *)(qp + 16 * t);
      if (qrow >= p.seq_q) qreg[rt][t] = bf16x8_t{};
    }
    qlimit[rt] = p.causal ? qrow + p.seq_offset : p.seq_kv;  // visible: key <= qlimit
  }

  const int wg_last = min(w.mt * WGROWS + WGROWS, p.seq_q) - 1;
  const int nblk = (key_end(p, wg_last) + BN - 1) / BN;
  const int wave_last = min(q_wave0 + WROWS - 1, p.seq_q - 1);
  const int ntw = (wave_last < q_wave0) ? 0 : (key_end(p, wave_last) + 31) / 32;  // tiles

  // register staging: 2 x 16 B per thread of a K block and of a V block,
  // rows crow and crow + 32 of the block; bytes past the last key row are
  // outside the descriptor's range and read as 0 (their scores are masked)
  const int crow = tid >> 3, ccol = (tid & 7) * 8;
  const int voff0 = (crow * (int)p.kv_rs + ccol) * 2, voff1 = voff0 + 64 * (int)p.kv_rs;
  u32x4_t k0, k1, v0, v1;
  // Every descriptor field goes through readfirstlane: the values are
  // uniform, but one computed on the VALU (the clamp) would leave the
  // descriptor in VGPRs and the compiler would wrap each load in a
  // readfirstlane/exec loop.
  auto rsrc = [&](const bf16_t *base, int blk) __attribute__((always_inline)) {
    const int rows = min(max(p.seq_kv - BN * blk, 0), BN);
    const uint64_t a = (uint64_t)(base + (int64_t)BN * blk * p.kv_rs);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    const int nrec = __builtin_amdgcn_readfirstlane(rows * (int)p.kv_rs * 2);
    return __builtin_amdgcn_make_buffer_rsrc((void *)(((uint64_t)hi << 32) | lo), (short)0, nrec,
                                             0x00020000);
  };
  auto gload_k = [&](int blk) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t r = rsrc(K, blk);
    k0 = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff0, 0, 0));
    k1 = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff1, 0, 0));
  };
  auto gload_v = [&](int blk) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t r = rsrc(V, blk);
    v0 = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff0, 0, 0));
    v1 = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff1, 0, 0));
  };
  auto lstore_k = [&](int buf) __attribute__((always_inline)) {
    bf16_t *ks = kring + buf * KBUF;
    *(u32x4_t *)(ks + crow * KP16 + ccol) = k0;
    *(u32x4_t *)(ks + (crow + 32) * KP16 + ccol) = k1;
  };
  auto lstore_v = [&](int buf) __attribute__((always_inline)) {
    bf16_t *vs = vring + buf * VBUF;
    *(u32x4_t *)(vs + crow * VP16 + ccol) = v0;
    *(u32x4_t *)(vs + (crow + 32) * VP16 + ccol) = v1;
  };

  float l[RT];    // row sum over both half-waves
  float mcv[RT];  // m * c: the reference max m (it moves only in the fixup) times c
  f32x16_t o[RT][2];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    mcv[rt] = -INFINITY;
    l[rt] = 0.f;
    o[rt][0] = f32x16_t{};
    o[rt][1] = f32x16_t{};
  }
  // Row-sum selector, the A operand of v_mfma_f32_16x16x32_bf16 (lane l holds
  // A[m = l%16][k = 8(l/16) .. +7]): A[m][k] = 1 where (m/4)%2 == (k/8)%2.
  // B = this step's P^T registers (lane l: 8 keys of query l%32), so D row m
  // sums the lanes whose query is the one D row m's lanes hold: every lane
  // receives the row sum of its own query over both half-waves.
  // (formed where it is used: four registers fewer across the loop)
  const uint32_t rs_bits = (((lane & 15) >> 2) & 1) == ((lane >> 4) & 1) ? 0x3f803f80u : 0u;
  const int tr_off = (4 * hf + ((lane & 15) >> 2)) * VP16 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  // --- pieces of a step
  auto kfrags = [&](const bf16_t *ks, bf16x8_t (&ka)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < 4; ++t) ka[t] = *(const bf16x8_t *)(ks + r32 * KP16 + 16 * t + 8 * hf);
  };
  // V^T fragments of the 32 keys at LDS rows vs: key slot j of 16-key chunk u
  // is key 16u + (j/4)*8 + 4hf + j%4, matching the S^T register order
  auto vfrags = [&](const bf16_t *vs, bf16x8_t (&va)[2][2]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const bf16_t *vsl = vs + 16 * u * VP16 + tr_off;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const bf16x4_t lo = tr16(vsl + 32 * dt);
        const bf16x4_t hi = tr16(vsl + 8 * VP16 + 32 * dt);
        va[u][dt] = bf16x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    }
  };
  auto scores = [&](const bf16x8_t (&ka)[4], f32x16_t (&s)[RT]) __attribute__((always_inline)) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      s[rt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[0], qreg[rt][0], f32x16_t{}, 0, 0, 0);
#pragma unroll
      for (int t = 1; t < 4; ++t)
        s[rt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[t], qreg[rt][t], s[rt], 0, 0, 0);
    }
  };
  auto pv = [&](const bf16x8_t (&va)[2][2], const bf16x8_t (&pb)[RT][2])
      __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
          o[rt][dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[u][dt], pb[rt][u], o[rt][dt], 0, 0, 0);
  };
  // p = exp2(s * c - mc) as bf16 MFMA operands (the row sum on the matrix cores)
  auto exps_p = [&](const f32x16_t &s, float mc, bf16x8_t (&pb)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int j = 0; j < 8; ++j) pb[u][j] = (__bf16)__builtin_amdgcn_exp2f(fmaf(s[8 * u + j], c, -mc));
  };
  // the row sum of a tile's bf16 P over both half-waves (D[0] once the MFMAs finish)
  auto rowsum = [&](const bf16x8_t (&pb)[2]) __attribute__((always_inline)) {
    uint32_t b = rs_bits;
    asm volatile("" : "+v"(b));  // keeps the selector from being hoisted out of the loop
    const bf16x8_t rs_sel = __builtin_bit_cast(bf16x8_t, u32x4_t{b, b, b, b});
    f32x4_t d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(rs_sel, pb[0], f32x4_t{}, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(rs_sel, pb[1], d, 0, 0, 0);
  };
  // p = exp2(s * c - mc) and the tile's row sum over both half-waves, read
  // as soon as its MFMAs finish (the fixup's exact path)
  auto exps = [&](const f32x16_t &s, float mc, bf16x8_t (&pb)[2], float &rs)
      __attribute__((always_inline)) {
    exps_p(s, mc, pb);
    rs = rowsum(pb)[0];
  };
  // causal / tail mask of tile t (keys kb..kb+31) in place
  auto mask = [&](int t, f32x16_t (&sc)[RT]) __attribute__((always_inline)) {
    const int kb = 32 * t;
    if (kb + 32 > p.seq_kv || (p.causal && kb + 31 > q_wave0 + p.seq_offset)) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = kb + (i >> 2) * 8 + hf * 4 + (i & 3);
          if (key >= p.seq_kv || key > qlimit[rt]) sc[rt][i] = -INFINITY;
        }
    }
  };
  // exact path for row tile rt (rare): move the reference max to the true
  // running max when it grew by more than 2^8 in probability (or was -inf),
  // rescale O and l, recompute P.  s holds raw scores, masked = -inf.
  auto fixup = [&](int rt, const f32x16_t &s, bf16x8_t (&pb)[2], float &rs)
      __attribute__((always_inline)) {
    float mx = s[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s[i]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    // in units of m*c: the true running max, moved to only when it grew by
    // more than 2^8 in probability (or nothing was visible yet)
    const float mt = fmaxf(mcv[rt], mx * c);  // -inf while nothing is visible
    const bool move = mcv[rt] == -INFINITY || mt - mcv[rt] > kRescaleLog2;
    const float m_new = move ? mt : mcv[rt];
    const float mn = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(mcv[rt] - mn);  // m = -inf -> 0
    l[rt] *= alpha;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[rt][dt][i] *= alpha;
    mcv[rt] = m_new;
    exps(s, mn, pb, rs);
  };
  // Row sums on the matrix cores: step t first settles tile t-1 -- its row
  // sum (rsp, from the MFMAs at the end of step t-1) is checked and, when a p
  // passed the limit (or is NaN), tile t-1 runs the fixup on its raw scores,
  // which are still in sn (not yet overwritten by tile t+1's scores), before
  // its P V; then the step's products, tile t's softmax into pc, and tile t's
  // row-sum MFMAs into rsc.  The softmax of the last step a wave runs is a
  // tile past its range (P = 0), so every real tile is settled.
  auto step = [&](auto masked_tag, int t, const bf16_t *vs, const bf16_t *ks, f32x16_t (&sc)[RT],
                      f32x16_t (&sn)[RT], bf16x8_t (&pp)[RT][2], bf16x8_t (&pc)[RT][2],
                      float (&rsp)[RT], float (&rsc)[RT]) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    {
      bool bad = false;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) bad = bad || !(rsp[rt] <= kSumLimit);
      if (__builtin_amdgcn_ballot_w64(bad) != 0) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) fixup(rt, sn[rt], pp[rt], rsp[rt]);
      }
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) l[rt] += rsp[rt];
    }
    if (!MASKED) {
    } else if (t >= ntw) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int i = 0; i < 16; ++i) sc[rt][i] = -INFINITY;
    } else {
      mask(t, sc);
    }
    bf16x8_t va[2][2], ka[4];
    vfrags(vs, va);
    kfrags(ks, ka);
    pv(va, pp);
    scores(ka, sn);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) exps_p(sc[rt], mcv[rt], pc[rt]);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) rsc[rt] = rowsum(pc[rt])[0];
    __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, kSchedV0, 0);
#pragma unroll
    for (int i = 0; i < 10 * RT; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, kSchedV1, 0);
    }
  };

  f32x16_t sa[RT], sb[RT];
  bf16x8_t pa[RT][2], pbb[RT][2];
  float rsa[RT], rsb[RT];  // row sums of the tiles in pa / pbb
  if (nblk > 0) {
    gload_k(0);
    gload_v(0);
    lstore_k(0);
    lstore_v(0);
    gload_k(1);
    gload_v(1);
    lstore_k(1);
    gload_k(2);
  }
  __syncthreads();
  if (ntw > 0) {  // step 0: scores of tiles 0 and 1, softmax of tile 0
    bf16x8_t ka[4];
    kfrags(kring, ka);
    scores(ka, sa);
    kfrags(kring + 32 * KP16, ka);
    scores(ka, sb);
    mask(0, sa);
    // first tile: the reference max starts at -inf, so the fast path always
    // ends in the fixup of every row tile; run the fixup directly (true max
    // first, one pass of exponentials instead of two) -- the same state
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float rs;
      fixup(rt, sa[rt], pa[rt], rs);
      rsa[rt] = rs;  // settled by step 1
    }
  }
  // iteration 0 stores K_2 into K_0's buffer, which step 0 reads: every wave
  // must be past those reads first
  __syncthreads();
  // iteration j: steps 2j+1 (P of tile 2j, scores of 2j+2, softmax of 2j+1)
  // and 2j+2 (P of 2j+1, scores of 2j+3, softmax of 2j+2).  The leading
  // iterations whose tiles every wave sees whole (no causal or tail mask)
  // run a step without any mask code.
  const int wg_first = w.mt * WGROWS;
  const int t_safe = max(0, p.causal ? min((wg_first + p.seq_offset + 1) / 32, p.seq_kv / 32)
                                     : p.seq_kv / 32);
  const int j_safe = min(nblk, max(0, (t_safe - 1) / 2));
  auto iteration = [&](auto masked_tag, int j) __attribute__((always_inline)) {
    const bf16_t *vc = vring + (j & 1) * VBUF;
    const bf16_t *kn = kring + ((j + 1) & 1) * KBUF;
    // masked iterations: a wave skips the steps past its causal range (step
    // ntw still adds P V of its last tile); the others' barriers and staging
    // go on, and the SIMD's other waves get the issue slots
    constexpr bool MASKED = decltype(masked_tag)::value;
    if (!MASKED || 2 * j + 1 <= ntw) step(masked_tag, 2 * j + 1, vc, kn, sb, sa, pa, pbb, rsa, rsb);
    if (!MASKED || 2 * j + 2 <= ntw)
      step(masked_tag, 2 * j + 2, vc + 32 * VP16, kn + 32 * KP16, sa, sb, pbb, pa, rsb, rsa);
    lstore_k(j & 1);        // K_{j+2} into K_j's buffer (K_j last read in iteration j-1)
    lstore_v((j + 1) & 1);  // V_{j+1} into V_{j-1}'s buffer
    gload_k(j + 3);         // rows past seq_kv read as 0
    gload_v(j + 2);
    __syncthreads();
  };
  int j = 0;
  for (; j < j_safe; ++j) iteration(std::false_type{}, j);
  for (; j < nblk; ++j) iteration(std::true_type{}, j);

#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int qrow = q_wave0 + row_step * rt + r32;
    const float lt = l[rt];  // the whole row's (both half-waves)
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;  // no visible key -> zeros
    if (p.lse && hf == 0 && qrow < p.seq_q)
      p.lse[((int64_t)w.b * p.n_heads + w.h + head_of(rt)) * p.seq_q + qrow] = row_lse(mcv[rt], lt);
    if (qrow < p.seq_q) {
      bf16_t *orow = O + (int64_t)head_of(rt) * HD + (int64_t)qrow * p.o_rs;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const int d0 = dt * 32 + gi * 8 + hf * 4;
          const uint32_t lo = (uint32_t)f32_to_bf16(o[rt][dt][4 * gi] * inv) |
                              ((uint32_t)f32_to_bf16(o[rt][dt][4 * gi + 1] * inv) << 16);
          const uint32_t hi = (uint32_t)f32_to_bf16(o[rt][dt][4 * gi + 2] * inv) |
                              ((uint32_t)f32_to_bf16(o[rt][dt][4 * gi + 3] * inv) << 16);
          *(uint2 *)(orow + d0) = make_uint2(lo, hi);
        }
    }
  }
}

// ------------------------------------------------------------------- fp32
constexpr int KP32 = HD + 4;  // 272 B pitch
constexpr int VP32 = BN + 4;

__global__ __launch_bounds__(256, 2) void prefill_f32_kernel(PrefillParams p) {
  // double-buffered K and V^T blocks: one barrier per block
  __shared__ __attribute__((aligned(16))) float Ks2[2][BN * KP32];
  __shared__ __attribute__((aligned(16))) float Vt2[2][HD * VP32];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r32 = lane & 31, hf = lane >> 5;
  // a (batch, KV head) group's heads and row tiles on one XCD: its K/V is
  // read from HBM once, then from that XCD's L2
  const Work w = decode_work_xcd(p);
  const float *Q = (const float *)p.q + w.b * p.q_bs + (int64_t)w.h * HD;
  const float *K = (const float *)p.k + w.b * p.kv_bs + (int64_t)w.g * HD;
  const float *V = (const float *)p.v + w.b * p.kv_bs + (int64_t)w.g * HD;
  float *O = (float *)p.o + w.b * p.o_bs + (int64_t)w.h * HD;

  const int q_wave0 = w.mt * BM + wave * 32;
  const int qrow = q_wave0 + r32;
  const bool row_ok = qrow < p.seq_q;

  // k-slot (hf, t) of the QK^T contraction is d = hf*32 + t
  float qreg[32];
#pragma unroll
  for (int t = 0; t < 32; t += 4) {
    float4 v4 = row_ok ? *(const float4 *)(Q + (int64_t)qrow * p.q_rs + hf * 32 + t)
                       : make_float4(0.f, 0.f, 0.f, 0.f);
    qreg[t] = v4.x; qreg[t + 1] = v4.y; qreg[t + 2] = v4.z; qreg[t + 3] = v4.w;
  }

  const int wg_last = min(w.mt * BM + BM, p.seq_q) - 1;
  const int kend = key_end(p, wg_last);
  const int nblk = (kend + BN - 1) / BN;
  const int wave_last = min(q_wave0 + 31, p.seq_q - 1);
  const int wave_kend = (wave_last < q_wave0) ? 0 : key_end(p, wave_last);
  const long qlimit = p.causal ? (long)qrow + p.seq_offset : (long)p.seq_kv;

  float4 kreg[4], vreg[4];
  auto gload = [&](int kb) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + 256 * c, key = idx >> 4, dc = idx & 15;
      const int kk = kb + key;
      if (kk < p.seq_kv) {
        kreg[c] = *(const float4 *)(K + (int64_t)kk * p.kv_rs + dc * 4);
        vreg[c] = *(const float4 *)(V + (int64_t)kk * p.kv_rs + dc * 4);
      } else {
        kreg[c] = make_float4(0.f, 0.f, 0.f, 0.f);
        vreg[c] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  };
  auto lstore = [&](int buf) {
    float *Ks = Ks2[buf], *Vt = Vt2[buf];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + 256 * c, key = idx >> 4, dc = idx & 15;
      *(float4 *)(Ks + key * KP32 + dc * 4) = kreg[c];
      Vt[(dc * 4 + 0) * VP32 + key] = vreg[c].x;
      Vt[(dc * 4 + 1) * VP32 + key] = vreg[c].y;
      Vt[(dc * 4 + 2) * VP32 + key] = vreg[c].z;
      Vt[(dc * 4 + 3) * VP32 + key] = vreg[c].w;
    }
  };

  float m = -INFINITY, l = 0.f;
  f32x16_t o[2] = {f32x16_t{}, f32x16_t{}};

  // block blk is computed from buffer blk & 1 while block blk + 1 (loaded
  // one block earlier) is stored into the other buffer, whose last reads were
  // in block blk - 1, before the previous barrier
  if (nblk > 0) {
    gload(0);
    lstore(0);
  }
  __syncthreads();
  if (nblk > 1) gload(BN);
  for (int blk = 0; blk < nblk; ++blk) {
    const int kb = blk * BN, buf = blk & 1;
    if (kb < wave_kend) {  // wave-uniform
      const float *Ks = Ks2[buf], *Vt = Vt2[buf];
    f32x16_t s[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      s[kt] = f32x16_t{};
      const float *krow = Ks + (kt * 32 + r32) * KP32 + hf * 32;
#pragma unroll
      for (int t = 0; t < 32; t += 4) {
        const float4 a = *(const float4 *)(krow + t);
        s[kt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, qreg[t], s[kt], 0, 0, 0);
        s[kt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, qreg[t + 1], s[kt], 0, 0, 0);
        s[kt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, qreg[t + 2], s[kt], 0, 0, 0);
        s[kt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, qreg[t + 3], s[kt], 0, 0, 0);
      }
    }
    const bool need_mask =
        (kb + BN > p.seq_kv) || (p.causal && (long)kb + BN - 1 > (long)q_wave0 + p.seq_offset);
    softmax_block(s, m, l, o, p.c, need_mask, kb, hf, qlimit, p.seq_kv);

    // register i of s[kt] is k-slot hf of key kt*32 + (i/4)*8 + hf*4 + i%4
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        const int kbase = kt * 32 + gi * 8 + hf * 4;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
          const float4 a = *(const float4 *)(Vt + (dt * 32 + r32) * VP32 + kbase);
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, s[kt][4 * gi], o[dt], 0, 0, 0);
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, s[kt][4 * gi + 1], o[dt], 0, 0, 0);
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, s[kt][4 * gi + 2], o[dt], 0, 0, 0);
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, s[kt][4 * gi + 3], o[dt], 0, 0, 0);
        }
      }
    }
    if (blk + 1 < nblk) {
      lstore(buf ^ 1);
      if (blk + 2 < nblk) gload(kb + 2 * BN);
    }
    __syncthreads();
  }

  const float lt = l + __shfl_xor(l, 32, 64);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  if (p.lse && hf == 0 && row_ok)
    p.lse[((int64_t)w.b * p.n_heads + w.h) * p.seq_q + qrow] = row_lse(m * p.c, lt);
  if (row_ok) {
    float *orow = O + (int64_t)qrow * p.o_rs;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        const int d0 = dt * 32 + gi * 8 + hf * 4;
        *(float4 *)(orow + d0) = make_float4(o[dt][4 * gi] * inv, o[dt][4 * gi + 1] * inv,
                                             o[dt][4 * gi + 2] * inv, o[dt][4 * gi + 3] * inv);
      }
  }
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace bn

using namespace bn;

static int prefill_impl(int dtype, const void *q, const void *k, const void *v, void *o,
                        int batch, int seq_q, int seq_kv, int n_heads, int n_kv_heads,
                        int head_dim, int64_t q_batch_stride, int64_t q_row_stride,
                        int64_t kv_batch_stride, int64_t kv_row_stride, int64_t o_batch_stride,
                        int64_t o_row_stride, float scale, int causal, int seq_offset,
                        float *lse, void *stream) {
  const char *op = "GQA prefill";
  if (dtype != BN_F32 && dtype != BN_BF16)
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": dtype must be F32 or BF16");
  if (batch < 0 || seq_q < 0 || seq_kv < 0)
    return fail(BN_ERR_SHAPE, std::string(op) + ": negative batch or sequence length");
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0)
    return fail(BN_ERR_SHAPE, std::string(op) + ": num_heads must be a positive multiple of num_kv_heads");
  if (head_dim != HD)
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": head_dim must be 64");
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(BN_ERR_INVALID_ARG, std::string(op) + ": scale must be positive and finite");
  if (batch == 0 || seq_q == 0) return BN_OK;
  if (!q || !o || (seq_kv > 0 && (!k || !v)))
    return fail(BN_ERR_INVALID_ARG, std::string(op) + ": NULL tensor pointer");
  if (q_row_stride < (int64_t)n_heads * HD || o_row_stride < (int64_t)n_heads * HD ||
      kv_row_stride < (int64_t)n_kv_heads * HD)
    return fail(BN_ERR_SHAPE, std::string(op) + ": row stride smaller than heads*head_dim");
  if (batch > 1 && (q_batch_stride < (int64_t)seq_q * q_row_stride ||
                    o_batch_stride < (int64_t)seq_q * o_row_stride ||
                    kv_batch_stride < (int64_t)seq_kv * kv_row_stride))
    return fail(BN_ERR_SHAPE, std::string(op) + ": batch stride smaller than seq*row_stride");
  const int64_t vec = dtype == BN_F32 ? 4 : 8;  // elements per 16 bytes
  if (!aligned16(q) || !aligned16(o) || (seq_kv > 0 && (!aligned16(k) || !aligned16(v))) ||
      q_row_stride % vec || kv_row_stride % vec || o_row_stride % vec || q_batch_stride % vec ||
      kv_batch_stride % vec || o_batch_stride % vec)
    return fail(BN_ERR_UNSUPPORTED,
                std::string(op) + ": pointers must be 16-byte aligned and strides multiples of 16 bytes");
  // bf16 K/V blocks are fetched through 32-bit buffer ranges of 64 rows
  if (dtype == BN_BF16 && kv_row_stride >= ((int64_t)1 << 24))
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": bf16 K/V row stride must be below 2^24 elements");
  // bf16: two 32-row tiles per wave (every LDS fragment feeds two MFMAs) when
  // that still leaves >= 1024 workgroups (4 per CU); one tile otherwise, so
  // small problems keep enough workgroups in flight (measured with settled
  // clocks: RT = 2 gains 3% on config 2 and 3-7% from S = 4096 on, and loses
  // 10-30% at 512 workgroups or fewer)
  constexpr int64_t kRt2MinWg = 1024;
  const int rt16 = ((int64_t)batch * n_heads * ((seq_q + 255) / 256) >= kRt2MinWg) ? 2 : 1;
  // bf16 with 4 or 8 query heads per KV head: head-packed work items (all of
  // a group's heads over 32 rows per workgroup; config 2 +6%, config 5 +3%)
  const int group = n_heads / n_kv_heads;
  const bool packed = dtype == BN_BF16 && (group == 8 || group == 4);
  const int rows_per_wg = packed ? 32 : dtype == BN_BF16 ? 4 * 32 * rt16 : BM;
  const int n_mt = (seq_q + rows_per_wg - 1) / rows_per_wg;
  const int64_t n_wg = (int64_t)batch * (packed ? n_kv_heads : n_heads) * n_mt;
  if (n_wg > 0x7fffffff) return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": problem too large");
  int st = ensure_device();
  if (st) return st;

  PrefillParams p;
  p.q = q; p.k = k; p.v = v; p.o = o;
  p.q_bs = q_batch_stride; p.q_rs = q_row_stride;
  p.kv_bs = kv_batch_stride; p.kv_rs = kv_row_stride;
  p.o_bs = o_batch_stride; p.o_rs = o_row_stride;
  p.batch = batch; p.seq_q = seq_q; p.seq_kv = seq_kv; p.n_heads = n_heads;
  p.group = n_heads / n_kv_heads; p.n_mt = n_mt;
  p.causal = causal ? 1 : 0; p.seq_offset = seq_offset;
  p.c = scale * 1.4426950408889634f;
  p.lse = lse;
  hipStream_t s = as_stream(stream);
  if (dtype == BN_BF16) {
    if (packed && group == 8)
      hipLaunchKernelGGL((prefill_bf16_kernel<2, kOcc, true>), dim3((unsigned)n_wg), dim3(256), 0, s, p);
    else if (packed)
      hipLaunchKernelGGL((prefill_bf16_kernel<1, kOcc, true>), dim3((unsigned)n_wg), dim3(256), 0, s, p);
    else if (rt16 == 2)
      hipLaunchKernelGGL((prefill_bf16_kernel<2, kOcc, false>), dim3((unsigned)n_wg), dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((prefill_bf16_kernel<1, kOcc, false>), dim3((unsigned)n_wg), dim3(256), 0, s, p);
  } else
    hipLaunchKernelGGL(prefill_f32_kernel, dim3((unsigned)n_wg), dim3(256), 0, s, p);
  BN_LAUNCH_CHECK();
  return BN_OK;
}

extern "C" int bn_gqa_prefill(int dtype, const void *q, const void *k, const void *v, void *o,
                              int batch, int seq_q, int seq_kv, int n_heads, int n_kv_heads,
                              int head_dim, int64_t q_batch_stride, int64_t q_row_stride,
                              int64_t kv_batch_stride, int64_t kv_row_stride,
                              int64_t o_batch_stride, int64_t o_row_stride, float scale,
                              int causal, int seq_offset, void *stream) {
  return prefill_impl(dtype, q, k, v, o, batch, seq_q, seq_kv, n_heads, n_kv_heads, head_dim,
                      q_batch_stride, q_row_stride, kv_batch_stride, kv_row_stride,
                      o_batch_stride, o_row_stride, scale, causal, seq_offset, nullptr, stream);
}

extern "C" int bn_gqa_prefill_lse(int dtype, const void *q, const void *k, const void *v, void *o,
                                  float *lse, int batch, int seq_q, int seq_kv, int n_heads,
                                  int n_kv_heads, int head_dim, int64_t q_batch_stride,
                                  int64_t q_row_stride, int64_t kv_batch_stride,
                                  int64_t kv_row_stride, int64_t o_batch_stride,
                                  int64_t o_row_stride, float scale, int causal, int seq_offset,
                                  void *stream) {
  if (!lse && batch > 0 && seq_q > 0)
    return fail(BN_ERR_INVALID_ARG, "GQA prefill: NULL log-sum-exp pointer");
  if (reinterpret_cast<uintptr_t>(lse) & 3u)
    return fail(BN_ERR_UNSUPPORTED, "GQA prefill: log-sum-exp pointer must be 4-byte aligned");
  return prefill_impl(dtype, q, k, v, o, batch, seq_q, seq_kv, n_heads, n_kv_heads, head_dim,
                      q_batch_stride, q_row_stride, kv_batch_stride, kv_row_stride,
                      o_batch_stride, o_row_stride, scale, causal, seq_offset, lse, stream);
}
