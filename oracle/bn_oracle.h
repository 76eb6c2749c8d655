/*
 * bn_oracle.h -- CPU restatement of BareNet's attention-path kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path and the timed CPU baseline in bench.py.  Only tests/, the smoke() entry
 * and bench.py's cpu_baseline leg may load it; the product library never
 * links, loads or falls back to it.
 *
 * Every function restates one reference kernel in its loop and reduction
 * order, on the reference's 2-D strided view (element (r,c) at
 * p[offset + r*stride_h + c*stride_w], src/utils/tensor.cuh:12).  Arithmetic
 * is fp32 with contraction disabled (-ffp-contract=off) so that the order of
 * operations is the one written here.
 *
 * Pinning (what checks each function, see tests/test_oracle.py):
 *   or_rmsnorm         closed form in fp64 (numpy, torch), rms(y)=1 invariant
 *   or_rope            fp64 complex-multiply restatement, norm preservation,
 *                      position-0 identity, relative-position invariant,
 *                      or_rope_backward inverse
 *   or_softmax         reference known-answer input [1,2,3,4] (test_llama.py:96),
 *                      fp64 closed form, masked entries exactly 0, rows sum to 1
 *   or_matmul          numpy fp64 matmul incl. transposed / sliced views
 *   or_repeat_kv       exact integer mapping test (constant-per-head values)
 *   or_gqa_prefill     torch.nn.functional.scaled_dot_product_attention
 *                      (enable_gqa) in fp64, Q=0 prefix-mean mask test,
 *                      brute-force fp64 loops
 *   or_gqa_decode      equals the last row of or_gqa_prefill; fp64 SDPA
 *   or_rmsnorm_rope    equals or_rope(or_rmsnorm(x)) bit-for-bit
 *   or_gqa_layer       numpy fp64 restatement of the layer op sequence
 *   backward kernels   finite differences / analytic fp64 gradients
 */
#ifndef BN_ORACLE_H
#define BN_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 2-D strided fp32 view, same fields as the reference Tensor<T> (tensor.cuh:45-50). */
typedef struct or_view {
  float *p;
  int64_t offset;
  int32_t h, w, stride_h, stride_w;
} or_view;

void or_rmsnorm(or_view x, or_view weight, or_view y, float eps);
void or_rmsnorm_backward(or_view x, or_view weight, or_view dy, or_view dx,
                         or_view dweight, float eps);
float or_rope_freq(int pair, int head_dim, float theta);
void or_rope(or_view x, or_view y, int position_offset, int head_dim, float theta);
void or_rope_backward(or_view dy, or_view dx, int position_offset, int head_dim,
                      float theta);
void or_rmsnorm_rope(or_view x, or_view weight, or_view y, float eps,
                     int position_offset, int head_dim, float theta);
void or_softmax(or_view x, or_view y, int causal, int seq_offset);
void or_softmax_backward(or_view y, or_view dy, or_view dx);
void or_matmul(or_view a, or_view b, or_view c);
void or_scale(or_view x, float c, or_view y);
void or_repeat_kv(or_view kv, or_view out, int head_dim, int n_rep);

/* Per-head causal GQA built from the reference primitives applied to column
 * slices: for each (b, h), O_h = softmax_causal(scale * Q_h K_g^T, off) V_g,
 * g = h / (n_heads / n_kv_heads).  Layout bshd: element (b, s, h, d) at
 * base[b*batch_stride + s*row_stride + h*head_dim + d].  scratch must hold
 * seq_q*seq_kv*2 floats. */
void or_gqa_prefill(const float *q, const float *k, const float *v, float *o,
                    int batch, int seq_q, int seq_kv, int n_heads,
                    int n_kv_heads, int head_dim, int64_t q_bs, int64_t q_rs,
                    int64_t kv_bs, int64_t kv_rs, int64_t o_bs, int64_t o_rs,
                    float scale, int causal, int seq_offset, float *scratch);

/* One query token per sequence, query position seq_lens[b]-1, keys
 * [0, seq_lens[b]).  q/o [B, H, D]; caches [B, max_len, Hkv, D].
 * scratch must hold max_len*2 floats. */
void or_gqa_decode(const float *q, const float *k_cache, const float *v_cache,
                   const int32_t *seq_lens, float *o, int batch, int max_len,
                   int n_heads, int n_kv_heads, int head_dim, float scale,
                   float *scratch);

/* The reference attention layer forward (llama_layers.hpp:57-113,
 * llama_layers.py:154-188) on one sequence: x [S, hidden] is the layer input
 * (already normalised by the caller, as in the decoder layer).  per_head = 0
 * reproduces the reference's fused-head chain (one S x S probability matrix
 * over the full hidden width); per_head = 1 uses or_gqa_prefill.
 * scratch must hold or_gqa_layer_scratch(...) floats. */
int64_t or_gqa_layer_scratch(int seq, int hidden, int n_heads, int n_kv_heads);
void or_gqa_layer(const float *x, int seq, int hidden, int n_heads,
                  int n_kv_heads, const float *wq, const float *wk,
                  const float *wv, const float *wo, float theta,
                  int position_offset, int per_head, float *out,
                  float *scratch);

#ifdef __cplusplus
}
#endif
#endif
