/*
 * bn_oracle.c -- CPU restatement of BareNet's attention-path kernels.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and CPU baseline); the product
 * never loads it.  Build: oracle/Makefile (gcc -O2 -ffp-contract=off).
 *
 * Each function names the reference kernel whose arithmetic it restates.
 * The reference launches 256-thread blocks for its row reductions; the
 * per-thread strided partials and the shared-memory tree (strides
 * 128, 64, ..., 1) are reproduced here so that fp32 rounding follows the
 * same association.
 */
#include "bn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define RED_THREADS 256

static inline float *at(or_view v, int r, int c) {
  return v.p + v.offset + (int64_t)r * v.stride_h + (int64_t)c * v.stride_w;
}

/* Shared-memory tree sum over 256 partials, strides 128 -> 1
 * (op_rmsnorm.cuh:36-41, op_softmax.cuh:59-64). */
static float tree_sum(float *s) {
  for (int stride = RED_THREADS / 2; stride > 0; stride >>= 1)
    for (int t = 0; t < stride; ++t) s[t] += s[t + stride];
  return s[0];
}

/* Tree max with the reference's strict '>' update (op_softmax.cuh:110-117). */
static float tree_max(float *s) {
  for (int stride = RED_THREADS / 2; stride > 0; stride >>= 1)
    for (int t = 0; t < stride; ++t)
      if (s[t + stride] > s[t]) s[t] = s[t + stride];
  return s[0];
}

/* op_rmsnorm_kernel, src/ops/op_rmsnorm.cuh:8-53. */
void or_rmsnorm(or_view x, or_view weight, or_view y, float eps) {
  float part[RED_THREADS];
  const int w = x.w;
  for (int r = 0; r < x.h; ++r) {
    for (int t = 0; t < RED_THREADS; ++t) {
      float s = 0.0f;
      for (int i = t; i < w; i += RED_THREADS) {
        float v = *at(x, r, i);
        s += v * v;
      }
      part[t] = s;
    }
    float mean_sq = tree_sum(part) / (float)w; /* :44 */
    float rms = sqrtf(mean_sq + eps);          /* :45 */
    for (int i = 0; i < w; ++i) {
      float normalized = *at(x, r, i) / rms;   /* :49, IEEE divide */
      *at(y, r, i) = normalized * *at(weight, 0, i);
    }
  }
}

/* op_rmsnorm_backward_kernel + host, src/ops/op_rmsnorm.cuh:55-133,161-187.
 * grad_weight is zero-filled first (:178); the device accumulates it with
 * atomicAdd in arbitrary row order, restated here in ascending row order. */
void or_rmsnorm_backward(or_view x, or_view weight, or_view dy, or_view dx,
                         or_view dweight, float eps) {
  float part[RED_THREADS];
  const int w = x.w;
  for (int i = 0; i < dweight.w; ++i) *at(dweight, 0, i) = 0.0f;
  for (int r = 0; r < x.h; ++r) {
    for (int t = 0; t < RED_THREADS; ++t) {
      float s = 0.0f;
      for (int i = t; i < w; i += RED_THREADS) {
        float v = *at(x, r, i);
        s += v * v;
      }
      part[t] = s;
    }
    float mean_sq = tree_sum(part) / (float)w;
    float rms = sqrtf(mean_sq + eps);
    float inv_rms = (float)(1.0 / (double)rms); /* :94, double literal */
    float inv_rms3 = inv_rms * inv_rms * inv_rms;
    for (int t = 0; t < RED_THREADS; ++t) {
      float s = 0.0f;
      for (int i = t; i < w; i += RED_THREADS)
        s += *at(dy, r, i) * *at(weight, 0, i) * *at(x, r, i);
      part[t] = s;
    }
    float sum_grad = tree_sum(part);
    for (int i = 0; i < w; ++i) {
      float xv = *at(x, r, i), g = *at(dy, r, i), wv = *at(weight, 0, i);
      float grad_norm = g * wv * inv_rms;
      float grad_rms = -inv_rms3 * xv * sum_grad / (float)w;
      *at(dx, r, i) = grad_norm + grad_rms;
      *at(dweight, 0, i) += g * (xv * inv_rms);
    }
  }
}

/* Rotation frequency of pair p, as formed in op_rope_kernel_simple
 * (src/ops/op_rope.cuh:82): exponent (float)(2p)/head_dim in fp32, theta^e
 * rounded to fp32, reciprocal taken in double (the literal 1.0) and rounded
 * to fp32.  theta^e is evaluated in double and rounded once. */
float or_rope_freq(int pair, int head_dim, float theta) {
  float e = (float)(2 * pair) / (float)head_dim;
  float p = (float)pow((double)theta, (double)e);
  return (float)(1.0 / (double)p);
}

static void rope_impl(or_view x, or_view y, int position_offset, int head_dim,
                      float theta, int inverse) {
  const int w = x.w;
  const int pairs = head_dim / 2;
  float *freq = (float *)malloc(sizeof(float) * (size_t)(pairs > 0 ? pairs : 1));
  for (int p = 0; p < pairs; ++p) freq[p] = or_rope_freq(p, head_dim, theta);
  for (int r = 0; r < x.h; ++r) {
    float pos = (float)(r + position_offset); /* :79 */
    for (int c = 0; c < w; ++c) {
      int head = c / head_dim, dih = c % head_dim;
      int p = dih / 2, odd = dih % 2;
      float angle = pos * freq[p];             /* :83, fp32 product */
      float ca = (float)cos((double)angle);
      float sa = (float)sin((double)angle);
      int base = head * head_dim + 2 * p;
      float x0 = *at(x, r, base), x1 = *at(x, r, base + 1);
      float out;
      if (!inverse)  /* op_rope.cuh:94-98 */
        out = odd ? x0 * sa + x1 * ca : x0 * ca - x1 * sa;
      else           /* op_rope.cuh:163-168 */
        out = odd ? -x0 * sa + x1 * ca : x0 * ca + x1 * sa;
      *at(y, r, c) = out;
    }
  }
  free(freq);
}

/* op_rope_kernel_simple, src/ops/op_rope.cuh:55-99. */
void or_rope(or_view x, or_view y, int position_offset, int head_dim, float theta) {
  rope_impl(x, y, position_offset, head_dim, theta, 0);
}

/* op_rope_backward_kernel, src/ops/op_rope.cuh:128-169. */
void or_rope_backward(or_view dy, or_view dx, int position_offset, int head_dim,
                      float theta) {
  rope_impl(dy, dx, position_offset, head_dim, theta, 1);
}

/* RMSNorm followed by RoPE on its output (the composition the fused kernel
 * replaces: llama_layers.py:157-163 with the norm of the decoder layer). */
void or_rmsnorm_rope(or_view x, or_view weight, or_view y, float eps,
                     int position_offset, int head_dim, float theta) {
  float *tmp = (float *)malloc(sizeof(float) * (size_t)x.h * (size_t)x.w);
  or_view t = {tmp, 0, x.h, x.w, x.w, 1};
  or_rmsnorm(x, weight, t, eps);
  or_rope(t, y, position_offset, head_dim, theta);
  free(tmp);
}

/* op_softmax_kernel / op_softmax_causal_kernel, src/ops/op_softmax.cuh:8-151. */
void or_softmax(or_view x, or_view y, int causal, int seq_offset) {
  float part[RED_THREADS];
  const int w = x.w;
  for (int r = 0; r < x.h; ++r) {
    long q = causal ? (long)r + seq_offset : (long)w; /* :89 */
    for (int t = 0; t < RED_THREADS; ++t) {
      float m = -INFINITY;
      for (int i = t; i < w; i += RED_THREADS)
        if (i <= q) {
          float v = *at(x, r, i);
          if (v > m) m = v;
        }
      part[t] = m;
    }
    float max_val = tree_max(part);
    for (int t = 0; t < RED_THREADS; ++t) {
      float s = 0.0f;
      for (int i = t; i < w; i += RED_THREADS) {
        if (i <= q) {
          float e = expf(*at(x, r, i) - max_val);
          *at(y, r, i) = e;
          s += e;
        } else {
          *at(y, r, i) = 0.0f; /* :129, masked entries are exactly 0 */
        }
      }
      part[t] = s;
    }
    float sum_val = tree_sum(part);
    for (int i = 0; i < w; ++i)
      if (i <= q) *at(y, r, i) = *at(y, r, i) / sum_val;
  }
}

/* op_softmax_backward_kernel, src/ops/op_softmax.cuh:182-224. */
void or_softmax_backward(or_view y, or_view dy, or_view dx) {
  float part[RED_THREADS];
  for (int r = 0; r < y.h; ++r) {
    for (int t = 0; t < RED_THREADS; ++t) {
      float s = 0.0f;
      for (int i = t; i < y.w; i += RED_THREADS) s += *at(y, r, i) * *at(dy, r, i);
      part[t] = s;
    }
    float sum = tree_sum(part);
    for (int i = 0; i < y.w; ++i)
      *at(dx, r, i) = *at(y, r, i) * (*at(dy, r, i) - sum);
  }
}

/* op_mm_tiled_kernel / op_mm_kernel (src/ops/op_mm_optimized.cuh:13-68,
 * src/ops/op_mm.cuh:23-36): one fp32 accumulator per output, k ascending. */
void or_matmul(or_view a, or_view b, or_view c) {
  for (int i = 0; i < c.h; ++i)
    for (int j = 0; j < c.w; ++j) {
      float s = 0.0f;
      for (int k = 0; k < a.w; ++k) s += *at(a, i, k) * *at(b, k, j);
      *at(c, i, j) = s;
    }
}

/* op_multiply(t, scalar), src/ops/op_elemwise.cuh:438-451. */
void or_scale(or_view x, float cval, or_view y) {
  for (int i = 0; i < x.h; ++i)
    for (int j = 0; j < x.w; ++j) *at(y, i, j) = *at(x, i, j) * cval;
}

/* repeat_kv, src/llama/llama_layers.hpp:131-175: destination head
 * kv_h*n_rep + r receives source head kv_h. */
void or_repeat_kv(or_view kv, or_view out, int head_dim, int n_rep) {
  int n_kv = kv.w / head_dim;
  for (int b = 0; b < kv.h; ++b)
    for (int g = 0; g < n_kv; ++g)
      for (int r = 0; r < n_rep; ++r)
        for (int d = 0; d < head_dim; ++d)
          *at(out, b, (g * n_rep + r) * head_dim + d) = *at(kv, b, g * head_dim + d);
}

void or_gqa_prefill(const float *q, const float *k, const float *v, float *o,
                    int batch, int seq_q, int seq_kv, int n_heads,
                    int n_kv_heads, int head_dim, int64_t q_bs, int64_t q_rs,
                    int64_t kv_bs, int64_t kv_rs, int64_t o_bs, int64_t o_rs,
                    float scale, int causal, int seq_offset, float *scratch) {
  const int group = n_heads / n_kv_heads;
  float *scores = scratch;
  float *probs = scratch + (int64_t)seq_q * seq_kv;
  for (int b = 0; b < batch; ++b)
    for (int h = 0; h < n_heads; ++h) {
      int g = h / group; /* llama_layers.hpp:159-163: head h reads KV head h/group */
      or_view Q = {(float *)q, b * q_bs + (int64_t)h * head_dim, seq_q, head_dim, (int32_t)q_rs, 1};
      or_view Kt = {(float *)k, b * kv_bs + (int64_t)g * head_dim, head_dim, seq_kv, 1, (int32_t)kv_rs};
      or_view V = {(float *)v, b * kv_bs + (int64_t)g * head_dim, seq_kv, head_dim, (int32_t)kv_rs, 1};
      or_view O = {o, b * o_bs + (int64_t)h * head_dim, seq_q, head_dim, (int32_t)o_rs, 1};
      or_view S = {scores, 0, seq_q, seq_kv, seq_kv, 1};
      or_view P = {probs, 0, seq_q, seq_kv, seq_kv, 1};
      or_matmul(Q, Kt, S);              /* query @ key.T  (llama_layers.py:174) */
      or_scale(S, scale, S);            /* * self.scale   (:177) */
      or_softmax(S, P, causal, seq_offset); /* (:180) */
      or_matmul(P, V, O);               /* @ value        (:183) */
    }
}

void or_gqa_decode(const float *q, const float *k_cache, const float *v_cache,
                   const int32_t *seq_lens, float *o, int batch, int max_len,
                   int n_heads, int n_kv_heads, int head_dim, float scale,
                   float *scratch) {
  const int64_t kv_rs = (int64_t)n_kv_heads * head_dim;
  for (int b = 0; b < batch; ++b) {
    int len = seq_lens[b];
    /* the new token is the last row of a prefill over len positions:
     * one query row at seq_offset len-1 sees keys [0, len). */
    or_gqa_prefill(q + (int64_t)b * n_heads * head_dim,
                   k_cache + (int64_t)b * max_len * kv_rs,
                   v_cache + (int64_t)b * max_len * kv_rs,
                   o + (int64_t)b * n_heads * head_dim, 1, 1, len, n_heads,
                   n_kv_heads, head_dim, 0, (int64_t)n_heads * head_dim, 0,
                   kv_rs, 0, (int64_t)n_heads * head_dim, scale, 1, len - 1,
                   scratch);
  }
}

int64_t or_gqa_layer_scratch(int seq, int hidden, int n_heads, int n_kv_heads) {
  int64_t kv = (int64_t)hidden / n_heads * n_kv_heads;
  int64_t s = seq;
  return s * hidden * 5 + s * kv * 3 + s * s * 2;
}

void or_gqa_layer(const float *x, int seq, int hidden, int n_heads,
                  int n_kv_heads, const float *wq, const float *wk,
                  const float *wv, const float *wo, float theta,
                  int position_offset, int per_head, float *out,
                  float *scratch) {
  const int D = hidden / n_heads;
  const int kvw = n_kv_heads * D;
  const int group = n_heads / n_kv_heads;
  const float scale = (float)(1.0 / sqrt((double)D)); /* llama_layers.hpp:54 */
  float *Q = scratch, *Qr = Q + (int64_t)seq * hidden;
  float *Krep = Qr + (int64_t)seq * hidden, *Vrep = Krep + (int64_t)seq * hidden;
  float *O = Vrep + (int64_t)seq * hidden;
  float *K = O + (int64_t)seq * hidden, *V = K + (int64_t)seq * kvw;
  float *Kr = V + (int64_t)seq * kvw;
  float *S = Kr + (int64_t)seq * kvw, *P = S + (int64_t)seq * seq;
  or_view X = {(float *)x, 0, seq, hidden, hidden, 1};
  or_view WQ = {(float *)wq, 0, hidden, hidden, hidden, 1};
  or_view WK = {(float *)wk, 0, hidden, kvw, kvw, 1};
  or_view WV = {(float *)wv, 0, hidden, kvw, kvw, 1};
  or_view WO = {(float *)wo, 0, hidden, hidden, hidden, 1};
  or_view vQ = {Q, 0, seq, hidden, hidden, 1}, vQr = {Qr, 0, seq, hidden, hidden, 1};
  or_view vK = {K, 0, seq, kvw, kvw, 1}, vKr = {Kr, 0, seq, kvw, kvw, 1};
  or_view vV = {V, 0, seq, kvw, kvw, 1};
  or_view vO = {O, 0, seq, hidden, hidden, 1};
  or_view vOut = {out, 0, seq, hidden, hidden, 1};
  or_matmul(X, WQ, vQ); /* llama_layers.hpp:73-75 */
  or_matmul(X, WK, vK);
  or_matmul(X, WV, vV);
  or_rope(vQ, vQr, position_offset, D, theta); /* :80-81 */
  or_rope(vK, vKr, position_offset, D, theta);
  if (!per_head) {
    or_view vKrep = {Krep, 0, seq, hidden, hidden, 1};
    or_view vVrep = {Vrep, 0, seq, hidden, hidden, 1};
    or_repeat_kv(vKr, vKrep, D, group); /* :87-89 */
    or_repeat_kv(vV, vVrep, D, group);
    or_view KT = {Krep, 0, hidden, seq, 1, hidden}; /* transpose view, :96 */
    or_view vS = {S, 0, seq, seq, seq, 1}, vP = {P, 0, seq, seq, seq, 1};
    or_matmul(vQr, KT, vS);                   /* :98 */
    or_scale(vS, scale, vS);                  /* :101 */
    or_softmax(vS, vP, 1, position_offset);   /* :105 */
    or_matmul(vP, vVrep, vO);                 /* :109 */
  } else {
    or_gqa_prefill(Qr, Kr, V, O, 1, seq, seq, n_heads, n_kv_heads, D, 0,
                   hidden, 0, kvw, 0, hidden, scale, 1, position_offset, S);
  }
  or_matmul(vO, WO, vOut); /* :112 */
}
