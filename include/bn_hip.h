/*
 * bn_hip.h -- C ABI of the MI355X (gfx950) attention-path library libbnhip.so.
 *
 * This is the boundary between host code (the pybind11 module `bten`, or any
 * FFI) and the HIP kernels.  Signatures carry plain pointers, sizes and POD
 * views only; no HIP, torch or C++ types cross it.  Every entry point returns
 * a bn_status; on failure bn_last_error() returns a thread-local message with
 * the same stem the reference throws as std::runtime_error (for example
 * "RMSNorm: weight shape must be (1, hidden_dim)", op_rmsnorm.cuh:146).
 * All arguments are validated on the host before anything is launched.
 *
 * Streams are opaque (`void *` holding a hipStream_t; NULL = the legacy
 * default stream, which is what the reference launches on).  Kernels are
 * asynchronous with respect to the host, like the reference's launches.
 *
 * Views: bn_view restates the reference's 2-D strided Tensor<T>
 * (src/utils/tensor.cuh:41-52): element (r, c) lives at
 * data[offset + r*stride_h + c*stride_w].  Transposes and slices are views
 * (tensor.cuh:133-171) and every op accepts them.
 */
#ifndef BN_HIP_H
#define BN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BN_ABI_VERSION 1

typedef enum bn_status {
  BN_OK = 0,
  BN_ERR_INVALID_ARG = 1, /* null pointer, bad enum, negative size */
  BN_ERR_SHAPE = 2,       /* shape mismatch, divisibility (reference runtime_error) */
  BN_ERR_UNSUPPORTED = 3, /* valid request outside what the kernels implement */
  BN_ERR_HIP = 4,         /* HIP runtime error: "HIP Error: <msg> (<code>) at file:line" */
  BN_ERR_OOM = 5,         /* memory pool could not satisfy an allocation */
  BN_ERR_NOT_DEVICE = 6   /* host tensor given to a GPU op ("only GPU implementation available") */
} bn_status;

typedef enum bn_dtype { BN_F32 = 0, BN_BF16 = 1, BN_U32 = 2 } bn_dtype;

typedef struct bn_view {
  void *data;        /* base of the allocation */
  int64_t offset;    /* element offset of element (0, 0) */
  int32_t h, w;      /* rows, columns */
  int32_t stride_h;  /* elements between rows */
  int32_t stride_w;  /* elements between columns */
  int32_t dtype;     /* bn_dtype */
  int32_t on_device; /* 1: device memory, 0: host memory */
} bn_view;

/* ------------------------------------------------------------------ runtime */
int bn_abi_version(void);
const char *bn_last_error(void);
/* Select the device and configure its stream-ordered pool.  Called implicitly
 * by the first allocation; explicit calls pick another device. */
int bn_init(int device);
int bn_device_count(int *count);
int bn_stream_create(void **stream);
int bn_stream_destroy(void *stream);
int bn_stream_synchronize(void *stream);
int bn_device_synchronize(void);
/* Free and total device memory of the library's device: replaces the
 * cudaMemGetInfo of LLaMAModel::get_gpu_memory_usage (llama_model.hpp:125-131). */
int bn_mem_get_info(size_t *free_bytes, size_t *total_bytes);

/* ------------------------------------------------------------- memory pool
 * Replaces CudaMemoryPool / PooledMemory (src/utils/memory_pool.cuh:15-125)
 * and the per-tensor cudaMalloc/cudaFree of Tensor<T> (tensor.cuh:15-26,
 * 59-77).  Allocations are stream-ordered (hipMallocAsync on the device's
 * memory pool with an unbounded release threshold), so a free never
 * synchronises the device; memory returns to the driver only through
 * bn_pool_trim. */
typedef struct bn_pool_stats {
  uint64_t bytes_in_use;      /* live bytes handed out (requested sizes) */
  uint64_t peak_bytes_in_use; /* high-water mark since the last reset */
  uint64_t bytes_reserved;    /* bytes the driver pool currently holds */
  uint64_t n_allocs;          /* successful bn_alloc calls */
  uint64_t n_frees;           /* successful bn_free calls */
  uint64_t n_live;            /* allocations not yet freed */
} bn_pool_stats;

int bn_alloc(void **ptr, size_t bytes, void *stream);
int bn_free(void *ptr, void *stream);
int bn_pool_get_stats(bn_pool_stats *out);
int bn_pool_reset_peak(void);
int bn_pool_trim(size_t min_bytes_to_keep);
/* Test hook: make allocations fail with BN_ERR_OOM once more than
 * `limit_bytes` are in use (0 = no limit). */
int bn_pool_set_limit(size_t limit_bytes);

/* kind: 0 host->device, 1 device->host, 2 device->device, 3 host->host.
 * Host<->device copies are synchronous with respect to the host, like
 * cudaMemcpy in Tensor::toHost/toDevice (tensor.cuh:80-131). */
int bn_memcpy(void *dst, const void *src, size_t bytes, int kind, void *stream);

/* --------------------------------------------------------------- path ops */
/* op_rmsnorm (src/ops/op_rmsnorm.cuh:135-159): y = x / sqrt(mean(x^2)+eps) * w.
 * x, y: [rows, hidden]; weight: [1, hidden].  F32 or BF16 (all the same). */
int bn_rmsnorm(const bn_view *x, const bn_view *weight, const bn_view *y,
               float eps, void *stream);
/* op_rmsnorm_backward (op_rmsnorm.cuh:161-187); dweight is overwritten. */
int bn_rmsnorm_backward(const bn_view *x, const bn_view *weight,
                        const bn_view *dy, const bn_view *dx,
                        const bn_view *dweight, float eps, void *stream);
/* op_rope (src/ops/op_rope.cuh:101-126): interleaved-pair rotation of every
 * head_dim-wide column block, position = row + position_offset. */
int bn_rope(const bn_view *x, const bn_view *y, int position_offset,
            int head_dim, float theta, void *stream);
/* op_rope_backward (op_rope.cuh:158-193). */
int bn_rope_backward(const bn_view *dy, const bn_view *dx, int position_offset,
                     int head_dim, float theta, void *stream);
/* No single reference counterpart: replaces op_rmsnorm followed by op_rope
 * on its output (one HBM read and one write instead of two each). */
int bn_rmsnorm_rope(const bn_view *x, const bn_view *weight, const bn_view *y,
                    float eps, int position_offset, int head_dim, float theta,
                    void *stream);
/* The decoder layer's residual add and the next RMSNorm in one pass
 * (llama_layers.hpp:241-272: x -> RMSNorm -> attention -> +x -> RMSNorm ->
 * MLP -> +x): h = x + delta, y = RMSNorm(h) * weight (op_rmsnorm
 * arithmetic).  h may alias x.  The reference's own fused kernel,
 * op_rmsnorm_residual (op_mm_optimized.cuh:93-162, unused there), adds the
 * residual after the norm; this is the pre-norm order the layer needs. */
int bn_add_rmsnorm(const bn_view *x, const bn_view *delta, const bn_view *weight,
                   const bn_view *h, const bn_view *y, float eps, void *stream);
/* SwiGLU activation: out = silu(gate) * up, silu(g) = g / (1 + exp(-g))
 * (op_silu.cuh:8-14 then op_multiply, llama_layers.hpp:199-211), one pass. */
int bn_silu_mul(const bn_view *gate, const bn_view *up, const bn_view *out, void *stream);
/* op_softmax (src/ops/op_softmax.cuh:153-180): row softmax; with causal,
 * column i of row r is kept iff i <= r + seq_offset, masked outputs are 0. */
int bn_softmax(const bn_view *x, const bn_view *y, int causal, int seq_offset,
               void *stream);
/* op_softmax_backward (op_softmax.cuh:226-246). */
int bn_softmax_backward(const bn_view *y, const bn_view *dy, const bn_view *dx,
                        void *stream);
/* op_mm (src/ops/op_mm.cuh:39-57): c = a @ b, fp32, any strides. */
int bn_matmul(const bn_view *a, const bn_view *b, const bn_view *c, void *stream);
/* Projection with RoPE in the epilogue: y = x @ w (x [M, K], w [K, N],
 * y [M, N], one dtype, BN_F32 or BN_BF16; rows contiguous and 16-byte
 * aligned, K and N multiples of 16 bytes), then op_rope's rotation (adjacent
 * pairs, freq = 1/theta^(2p/head_dim), position = position_offset + row) on
 * columns [0, rope_cols), a multiple of head_dim (0: no rotation).  Replaces
 * op_mm for the Q, K and V projections followed by op_rope on Q and K
 * (llama_layers.hpp:72-81) -- one call on the concatenated weight
 * [hidden, (H + 2*Hkv)*head_dim] with rope_cols = (H + Hkv)*head_dim -- and
 * op_mm for the output projection (:112, rope_cols = 0).  fp32 accumulation;
 * y must not overlap x or w.  Split-k partial sums take
 * bn_linear_rope_workspace_size(dtype, M, N, K) bytes of workspace (16-byte
 * aligned; NULL: the pool supplies them).  w may also be output-major -- the
 * transposed view of an [N, K] matrix (stride_h 1, stride_w a multiple of 16
 * bytes, the view's element (0, 0) 16-byte aligned): for M <= 4 and
 * M*ceil(K / (64*elements per 16 bytes))*64*elements per 16 bytes <= 16384
 * this streams each output's contiguous weights once with no k split (no
 * workspace; N even; x rows 16-byte aligned, y rows contiguous at any
 * stride); fp32 with more rows runs a matrix-core kernel of 32 x 128 output
 * tiles (no workspace, no k split); bf16 with more than 4 rows is
 * BN_ERR_UNSUPPORTED for that layout. */
size_t bn_linear_rope_workspace_size(int dtype, int m, int n, int k);
int bn_linear_rope(const bn_view *x, const bn_view *w, const bn_view *y,
                   int rope_cols, int position_offset, int head_dim, float theta,
                   void *workspace, size_t workspace_bytes, void *stream);
/* repeat_kv (src/llama/llama_layers.hpp:131-175, llama_layers.py:105-138):
 * out column block kv_h*n_rep + r = kv column block kv_h, on the device. */
int bn_repeat_kv(const bn_view *kv, const bn_view *out, int head_dim, int n_rep,
                 void *stream);
/* The fused-head attention chain of src/llama/llama_layers.hpp:83-109 in one
 * launch: with n_rep = n_heads / n_kv_heads and K_rep / V_rep = repeat_kv(k /
 * v, n_rep) (head h reads KV head h / n_rep),
 *   o = softmax((q @ K_rep^T) * scale, causal, seq_offset) @ V_rep
 * -- ONE probability matrix over the full n_heads*head_dim-wide rows, as the
 * reference's op_mm / op_multiply / op_softmax / op_mm chain computes it --
 * without forming K_rep, V_rep or the seq_q x seq_kv matrices.
 * q, o: [seq_q, n_heads*head_dim]; k, v: [seq_kv, n_kv_heads*head_dim]; fp32
 * views whose columns are contiguous and whose rows start on 16-byte
 * boundaries.  Causal mask as op_softmax.cuh:89-99 (key j is visible to row i
 * iff j <= i + seq_offset); a row with no visible key is written as zeros, as
 * the chain's all-zero probability row gives.  Needs head_dim % 4 == 0 and
 * n_kv_heads*head_dim a multiple of 16, at most 512.  Results agree with the
 * chain to fp32 rounding (the sums associate differently).  From 512 rows of
 * q with n_kv_heads*head_dim = 256 the call runs on the matrix cores in three
 * launches and takes a stream-ordered pool allocation for the group sums of q
 * and the key blocks' records (seq_q*1 KB plus ~33 KB per 32 x 128 block),
 * released on the same stream; shorter prompts take one launch and no
 * memory. */
int bn_fused_head_attention(const bn_view *q, const bn_view *k, const bn_view *v,
                            const bn_view *o, int n_heads, int n_kv_heads,
                            int head_dim, float scale, int causal, int seq_offset,
                            void *stream);

/* Elementwise surface used by the layers (src/ops/op_elemwise.cuh:326-507,
 * op_silu.cuh, op_reduction.cuh).  Binary ops broadcast b along a unit
 * dimension as op_elemwise_binary_w_bcast_kernel does (:221-243). */
typedef enum bn_binop { BN_ADD = 0, BN_SUB = 1, BN_MUL = 2, BN_EQ = 3 } bn_binop;
typedef enum bn_unop {
  BN_RELU = 0, BN_SILU = 1, BN_ADD_SCALAR = 2, BN_MUL_SCALAR = 3
} bn_unop;
typedef enum bn_gradop { BN_RELU_BACK = 0, BN_SILU_BACK = 1 } bn_gradop;
int bn_binary(int op, const bn_view *a, const bn_view *b, const bn_view *y,
              void *stream);
int bn_unary(int op, const bn_view *x, float scalar, const bn_view *y,
             void *stream);
int bn_unary_backward(int op, const bn_view *x, const bn_view *dy,
                      const bn_view *dx, void *stream);
/* op_const_fill; value is reinterpreted for U32 views. */
int bn_fill(const bn_view *y, double value, void *stream);
/* op_uniform_fill (op_elemwise.cuh:487-507; cuRAND there): values uniform in
 * [lo, hi] (F32 or BF16), element (i, j) from a counter-based generator
 * (SplitMix64) of seed and the logical index i*w + j, so the result does not
 * depend on strides, launch shape or device. */
int bn_fill_uniform(const bn_view *y, float lo, float hi, uint64_t seed, void *stream);
/* LLaMAModel::embed (llama_model.hpp:161-198): out row r = table row ids[r];
 * ids device uint32 [n]; table [vocab, hidden] and out [n, hidden] of one
 * dtype (F32 or BF16).  An id >= vocab gives a zero row. */
int bn_embedding(const bn_view *table, const uint32_t *ids, int n, const bn_view *out,
                 void *stream);
/* op_sum (axis 0 -> [1, w], axis 1 -> [h, 1]) and op_argmax (row-wise, U32). */
int bn_sum(const bn_view *x, const bn_view *y, int axis, void *stream);
int bn_argmax(const bn_view *x, const bn_view *y, void *stream);
/* Converting copy between views of the same shape (F32 <-> BF16, same dtype). */
int bn_copy(const bn_view *x, const bn_view *y, void *stream);

/* ----------------------------------------------------- fused GQA attention
 * No single reference counterpart: replaces the per-head chain
 *   Q_h @ K_g^T (op_mm) -> * scale (op_multiply) -> op_softmax(causal,
 *   seq_offset) -> @ V_g (op_mm),       g = h / (n_heads / n_kv_heads)
 * (llama_layers.py:174-183 / llama_layers.hpp:96-109 applied per head,
 * repeat_kv mapping of llama_layers.hpp:159-163).
 *
 * Layout "bshd": element (b, s, head, d) at base[b*batch_stride +
 * s*row_stride + head*head_dim + d], strides in elements; the reference's
 * [S, heads*head_dim] row per token is the b = 0 slice.  dtype is BN_F32 or
 * BN_BF16 for q, k, v and o alike; accumulation is fp32.  head_dim must be 64.
 * With causal, key j is visible to query row i iff j <= i + seq_offset
 * (op_softmax.cuh:89-99); a row with no visible key produces zeros. */
int bn_gqa_prefill(int dtype, const void *q, const void *k, const void *v,
                   void *o, int batch, int seq_q, int seq_kv, int n_heads,
                   int n_kv_heads, int head_dim, int64_t q_batch_stride,
                   int64_t q_row_stride, int64_t kv_batch_stride,
                   int64_t kv_row_stride, int64_t o_batch_stride,
                   int64_t o_row_stride, float scale, int causal,
                   int seq_offset, void *stream);
/* bn_gqa_prefill that also writes, per (batch, query head, row), the natural
 * log of the row's softmax denominator, lse = log sum_{visible j}
 * exp(scale * q_i . k_j) (-inf for a row with no visible key), into lse
 * [batch, n_heads, seq_q] fp32 contiguous: the residual the backward needs.
 * No reference counterpart as one call (the reference's autograd keeps the
 * probability matrix instead). */
int bn_gqa_prefill_lse(int dtype, const void *q, const void *k, const void *v,
                       void *o, float *lse, int batch, int seq_q, int seq_kv,
                       int n_heads, int n_kv_heads, int head_dim,
                       int64_t q_batch_stride, int64_t q_row_stride,
                       int64_t kv_batch_stride, int64_t kv_row_stride,
                       int64_t o_batch_stride, int64_t o_row_stride, float scale,
                       int causal, int seq_offset, void *stream);

/* Backward of bn_gqa_prefill (bf16, head_dim 64), flash-style: with
 * P = exp(scale * Q_h K_g^T - lse) over the visible keys (g = h / (n_heads /
 * n_kv_heads)), dP = dO_h V_g^T and D = rowsum(dO_h * O_h),
 *   dq_h = scale * (P * (dP - D)) K_g
 *   dk_g = scale * sum over the heads h of group g of (P * (dP - D))^T Q_h
 *   dv_g = sum over the heads h of group g of P^T dO_h
 * q/dq share (q_batch_stride, q_row_stride), o/dout share the o strides,
 * k/v/dk/dv share the kv strides ("bshd" layout as bn_gqa_prefill); lse is
 * bn_gqa_prefill_lse's output [batch, n_heads, seq_q].  causal / seq_offset
 * as in the forward.  dq, dk and dv are written, not accumulated.  It
 * replaces the reference autograd chain through op_mm (op_mm.cuh),
 * op_softmax_backward (op_softmax.cuh:182-246), the scale op and repeat_kv's
 * gradient sum (llama_layers.hpp:156-167).  workspace (16-byte aligned,
 * bn_gqa_prefill_backward_workspace_size bytes: fp32 D and, when a KV head's
 * query heads are split over workgroups, fp32 dK/dV partial sums) may be
 * NULL: the pool then supplies it.  Results are deterministic: no atomics. */
size_t bn_gqa_prefill_backward_workspace_size(int batch, int seq_q, int seq_kv,
                                              int n_heads, int n_kv_heads,
                                              int head_dim, int causal);
int bn_gqa_prefill_backward(int dtype, const void *q, const void *k,
                            const void *v, const void *o, const void *dout,
                            const float *lse, void *dq, void *dk, void *dv,
                            int batch, int seq_q, int seq_kv, int n_heads,
                            int n_kv_heads, int head_dim,
                            int64_t q_batch_stride, int64_t q_row_stride,
                            int64_t kv_batch_stride, int64_t kv_row_stride,
                            int64_t o_batch_stride, int64_t o_row_stride,
                            float scale, int causal, int seq_offset,
                            void *workspace, size_t workspace_bytes,
                            void *stream);

/* ------------------------------------------------------- decode driver
 * Greedy decode of a LLaMA-style decoder (pre-norm GQA attention + SwiGLU
 * MLP, llama_layers.hpp:241-272; fp32, head_dim 64) with per-layer KV caches
 * [max_len, n_kv_heads*64].  Step t processes token t (first_token for t = 0,
 * else tokens_out[t-1]) at position `position + t`: embedding row, every layer
 * (QKV projection with RoPE, K/V appended to the caches at that row,
 * bn_gqa_decode over the cache, O projection, residual add + RMSNorm, gate|up
 * projection, SwiGLU, down projection, residual add + RMSNorm), lm_head, and
 * writes the argmax of the logits to tokens_out[t] (device, uint32).  Nothing
 * waits for the host between steps.  Replaces the reference's generate loop
 * (llama_model.py:112-168), which has no cache and reruns the prefix per
 * token (:135-141); the reference samples from softmax(logits / T) with an
 * optional top-k and stops at eos_token_id (:145-162), this loop is its
 * deterministic limit (top_k = 1, argmax) and runs all n steps.  Weight layouts are x @ W: wqkv [hidden, (H + 2*Hkv)*64]
 * (Q | K | V), wo [hidden, hidden], wgu [hidden, 2*intermediate] (gate | up),
 * wd [intermediate, hidden], embed [vocab, hidden], lm_head [hidden, vocab];
 * norm weights [hidden].  With weights_out_major set, wqkv, wo, wgu, wd and
 * lm_head are stored transposed ([out, in] row-major: each output's weights
 * contiguous), and every projection streams them without a k split (see
 * bn_linear_rope); with hidden <= 2048 each RMSNorm (and the residual add
 * before it) is then formed inside the projection that reads it, with the
 * arithmetic of bn_rmsnorm / bn_add_rmsnorm (same tokens and caches, 44 fewer
 * launches per step on TinyLLaMA).  workspace (256-byte aligned,
 * bn_llama_decode_workspace_size bytes) may be NULL: the pool supplies it. */
typedef struct bn_llama_config {
  int n_layers, hidden, n_heads, n_kv_heads, intermediate, vocab, max_len;
  float rms_eps, rope_theta;
  int weights_out_major;  /* 0: [in, out] row-major (x @ W); 1: [out, in] row-major */
} bn_llama_config;
typedef struct bn_llama_layer_weights {
  const float *ln1, *wqkv, *wo, *ln2, *wgu, *wd;
  float *k_cache, *v_cache;
} bn_llama_layer_weights;
size_t bn_llama_decode_workspace_size(const bn_llama_config *config);
int bn_llama_decode(const bn_llama_config *config, const float *embed,
                    const float *ln_f, const float *lm_head,
                    const bn_llama_layer_weights *layers, int first_token,
                    int position, int n_tokens, uint32_t *tokens_out,
                    void *workspace, size_t workspace_bytes, void *stream);

/* KV-cache decode: one new query token per sequence.  The reference has no
 * KV cache (llama_model.py:135-141 recomputes the prefix); this is the last
 * row of bn_gqa_prefill with seq_offset = seq_lens[b]-1 over keys
 * [0, seq_lens[b]).  q, o: [batch, n_heads, head_dim] contiguous; caches:
 * [batch, max_len, n_kv_heads, head_dim] contiguous; seq_lens: device int32
 * [batch], each in [1, max_len] (read on the device: a length <= 0 gives a
 * zero output row, a length above max_len is treated as max_len, i.e. the
 * whole cache is attended).  workspace: device memory of
 * bn_gqa_decode_workspace_size() bytes (NULL: taken from the pool when the
 * call needs it); single-pass calls use none: bf16 caches with
 * batch*n_kv_heads >= the device's compute units.  fp32 caches of at most
 * 1024 keys with batch*n_heads <= 256 keep 4 split records per (sequence,
 * head) in it and merge them in the same launch, counting on a ring of 16
 * counter slots inside the library: at most 16 such calls in flight at once
 * on one GPU (more would share a slot and race). */
size_t bn_gqa_decode_workspace_size(int batch, int max_len, int n_heads,
                                    int head_dim);
int bn_gqa_decode(int dtype, const void *q, const void *k_cache,
                  const void *v_cache, const int32_t *seq_lens, void *o,
                  int batch, int max_len, int n_heads, int n_kv_heads,
                  int head_dim, float scale, void *workspace,
                  size_t workspace_bytes, void *stream);

/* bn_gqa_decode over caches of any layout whose key rows are head_dim
 * contiguous elements: element k of key row j of KV head g of sequence b is
 * cache[b*cache_seq_stride + g*cache_head_stride + j*cache_row_stride + k]
 * (strides in elements, positive multiples of 16 bytes; K and V share them).
 * The same row of the reference as bn_gqa_decode (the last row of the causal
 * softmax, op_softmax.cuh:89-99, over the prefix llama_model.py:135-141
 * recomputes); the reference keeps no cache, so its layout is this library's
 * choice.  bn_gqa_decode is this call with the contiguous
 * [batch, max_len, n_kv_heads, head_dim] strides (max_len*n_kv_heads*head_dim,
 * head_dim, n_kv_heads*head_dim).  A head-major [batch, n_kv_heads, max_len,
 * head_dim] cache (n_kv_heads*max_len*head_dim, max_len*head_dim, head_dim)
 * keeps each (sequence, KV head)'s rows contiguous in HBM and streams faster
 * on bf16 caches of at least one (sequence, KV head) per compute unit.  Same
 * kernels, workspace and results as bn_gqa_decode on the same values, except
 * that when a KV head's rows are contiguous (cache_row_stride == head_dim),
 * bf16 caches of at least one (sequence, KV head) per compute unit in batches
 * of at most 512 stream a cache longer than 1.25x the batch's mean length
 * with six waves instead of four: the same row to the bf16 tolerance, summed
 * in another order. */
int bn_gqa_decode_strided(int dtype, const void *q, const void *k_cache,
                          const void *v_cache, const int32_t *seq_lens, void *o,
                          int batch, int max_len, int n_heads, int n_kv_heads,
                          int head_dim, int64_t cache_seq_stride,
                          int64_t cache_head_stride, int64_t cache_row_stride,
                          float scale, void *workspace, size_t workspace_bytes,
                          void *stream);

/* bn_gqa_decode with the lengths also on the host (h_seq_lens: host int32
 * [batch], the values seq_lens holds on the device), as a serving loop has
 * them.  Replaces the same row as bn_gqa_decode (the last row of the causal
 * softmax, op_softmax.cuh:89-99, over the cache llama_model.py:135-141
 * recomputes).  From the host lengths the call plans equal shares of the
 * batch's 32-key tiles, one per compute unit, so a ragged batch's long caches
 * are cut across several workgroups and merged in the same launch instead of
 * streaming alone at the end; bf16 caches, 1/2/4/8 query heads per KV head,
 * at least as many (sequence, KV head) units as compute units (at most 256)
 * and a longest cache above 1.25x the mean.  Every other call (a balanced
 * batch included) runs bn_gqa_decode on seq_lens.  workspace: device memory of
 * bn_gqa_decode_planned_workspace_size() bytes, or NULL (the pool); calls in
 * flight at once need workspaces of their own (each launch tags the records
 * it writes there with its own epoch; nothing else is shared). */
size_t bn_gqa_decode_planned_workspace_size(int batch, int max_len, int n_heads,
                                            int n_kv_heads, int head_dim);
int bn_gqa_decode_planned(int dtype, const void *q, const void *k_cache,
                          const void *v_cache, const int32_t *seq_lens,
                          const int32_t *h_seq_lens, void *o, int batch,
                          int max_len, int n_heads, int n_kv_heads, int head_dim,
                          float scale, void *workspace, size_t workspace_bytes,
                          void *stream);

/* bn_gqa_decode_planned over caches of any layout whose key rows are contiguous
 * (strides as for bn_gqa_decode_strided; the unplanned fallback is
 * bn_gqa_decode_strided).  Same reference row; the plan and kernel are the
 * planned call's. */
int bn_gqa_decode_planned_strided(int dtype, const void *q, const void *k_cache,
                                  const void *v_cache, const int32_t *seq_lens,
                                  const int32_t *h_seq_lens, void *o, int batch,
                                  int max_len, int n_heads, int n_kv_heads,
                                  int head_dim, int64_t cache_seq_stride,
                                  int64_t cache_head_stride,
                                  int64_t cache_row_stride, float scale,
                                  void *workspace, size_t workspace_bytes,
                                  void *stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): bn_gqa_decode with the same arguments, kernels and
 * results, minus the workspace.  Its split-K chunk partials live in a
 * file-scope device array of BN_GQA_DECODE_SCRATCH_BYTES per GPU (held until
 * the process ends; its address is looked up once per device by bn_init).
 * It calls no hipMalloc, hipFree or pool allocation; a call whose partials
 * would exceed the array fails with BN_ERR_UNSUPPORTED before any device
 * work.  Every call on one GPU shares that GPU's array and leaves its last
 * contents there (nothing needs clearing: each call writes every record it
 * reads; the short-cache split's counters return to zero at the end of each
 * launch), so calls that overlap on one GPU -- on different streams, or from
 * different threads -- race; serialise them. */
#define BN_GQA_DECODE_SCRATCH_BYTES (32u << 20)
int bn_gqa_decode_noalloc(int dtype, const void *q, const void *k_cache,
                          const void *v_cache, const int32_t *seq_lens, void *o,
                          int batch, int max_len, int n_heads, int n_kv_heads,
                          int head_dim, float scale, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* BN_HIP_H */
