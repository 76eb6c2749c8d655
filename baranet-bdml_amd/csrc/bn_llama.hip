// bn_llama.hip -- greedy decode of a LLaMA-style decoder (TinyLLaMA's
// layout: pre-norm GQA attention + SwiGLU MLP, fp32) with per-layer KV caches,
// driven from the host without a synchronisation per token: each step's
// token stays on the device, where the next step's embedding gather reads it.
// The reference has no KV cache and reruns the whole prefix for every token
// (llama_model.py:135-141, llama_model.hpp:161-198); its decoder layer is
// llama_layers.hpp:241-272.  Every step is the path's own kernels:
// bn_linear_rope's projections (the QKV rotation and the K/V cache append in
// their epilogue; the SwiGLU product in the gate|up projection's),
// bn_gqa_decode, bn_add_rmsnorm, bn_rmsnorm and bn_argmax.  The fused
// epilogues see the sums the unfused projection writes (the split-k slabs in
// one order; with output-major weights each output's own dot product), so
// the tokens and caches are those of the op-by-op step loop.  With
// output-major weights the RMSNorms (and the residual adds before them) are
// formed in the x staging of the projection that reads them, with the norm
// kernels' arithmetic: 113 launches per step instead of 158, the same bits.
#include <algorithm>

#include "bn_common.hpp"

namespace bn {
namespace {

// x = embed[token]; the token comes from `tok` (device) or, when tok is
// null, from `first`; ids past the table are clamped (argmax never gives one).
// vec (a 16-byte aligned table; hidden is a multiple of 4): 16-byte chunks,
// all of a thread's requested before any is stored
__global__ __launch_bounds__(256) void embed_gather_kernel(const float *embed, const uint32_t *tok,
                                                           uint32_t first, int vocab, float *x,
                                                           int hidden, int vec) {
  uint32_t t = tok ? *tok : first;
  t = t < (uint32_t)vocab ? t : (uint32_t)(vocab - 1);
  const float *row = embed + (int64_t)t * hidden;
  if (!vec) {
    for (int i = threadIdx.x; i < hidden; i += 256) x[i] = row[i];
    return;
  }
  constexpr int U = 4;
  const int n4 = hidden / 4;
  for (int c0 = threadIdx.x; c0 < n4; c0 += 256 * U) {
    float4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = ((const float4 *)row)[min(c0 + 256 * u, n4 - 1)];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (c0 + 256 * u < n4) ((float4 *)x)[c0 + 256 * u] = v[u];
  }
}

// out row r = table row ids[r] (one workgroup per row); an id outside the
// table gives a zero row
template <typename T>
__global__ __launch_bounds__(256) void embed_rows_kernel(DView<const T> table, const uint32_t *ids,
                                                         DView<T> out) {
  const int r = blockIdx.x;
  const uint32_t id = ids[r];
  const bool ok = id < (uint32_t)table.h;
  for (int j = threadIdx.x; j < out.w; j += 256)
    out.at(r, j) = ok ? table.at((int)id, j) : T(0);
}

// lens[i] = first + i + 1 (the cache length after step i)
__global__ __launch_bounds__(256) void fill_lens_kernel(int32_t *lens, int first, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) lens[i] = first + i + 1;
}

bn_view fview(const void *p, int h, int w, int stride_h) {
  bn_view v;
  v.data = const_cast<void *>(p);
  v.offset = 0;
  v.h = h;
  v.w = w;
  v.stride_h = stride_h;
  v.stride_w = 1;
  v.dtype = BN_F32;
  v.on_device = 1;
  return v;
}

// the [in, out] view of a projection weight: row-major, or the transposed
// view of an output-major [out, in] matrix
bn_view wview(const void *p, int in, int out, bool out_major) {
  bn_view v = fview(p, in, out, out);
  if (out_major) {
    v.stride_h = 1;
    v.stride_w = in;
  }
  return v;
}

size_t a256(size_t n) { return (n + 255) & ~(size_t)255; }

// workspace regions, in bytes from the start
struct Plan {
  size_t hdn, hdn2, xn, qkv, o, attn, act, mlp, logits, tok, lens, lin, dec, total;
  size_t lin_bytes, dec_bytes;
};

Plan plan_of(const bn_llama_config *c) {
  const int hd = c->hidden / c->n_heads, kv = c->n_kv_heads * hd;
  const int shapes[5][2] = {{c->hidden, c->hidden + 2 * kv}, {c->hidden, c->hidden},
                            {c->hidden, 2 * c->intermediate}, {c->intermediate, c->hidden},
                            {c->hidden, c->vocab}};
  size_t lin = 0;
  for (const auto &s : shapes) lin = std::max(lin, bn_linear_rope_workspace_size(BN_F32, 1, s[1], s[0]));
  Plan p;
  size_t at = 0;
  auto take = [&](size_t bytes) { const size_t r = at; at += a256(bytes); return r; };
  p.hdn = take(4 * (size_t)c->hidden);
  p.hdn2 = take(4 * (size_t)c->hidden);
  p.xn = take(4 * (size_t)c->hidden);
  p.qkv = take(4 * (size_t)(c->hidden + 2 * kv));
  p.o = take(4 * (size_t)c->hidden);
  p.attn = take(4 * (size_t)c->hidden);
  p.act = take(4 * (size_t)c->intermediate);
  p.mlp = take(4 * (size_t)c->hidden);
  p.logits = take(4 * (size_t)c->vocab);
  p.tok = take(4);
  p.lens = take(4 * (size_t)c->max_len);
  p.lin_bytes = lin;
  p.lin = take(lin);
  p.dec_bytes = bn_gqa_decode_workspace_size(1, c->max_len, c->n_heads, hd);
  p.dec = take(p.dec_bytes);
  p.total = at;
  return p;
}

int check_config(const bn_llama_config *c) {
  const char *op = "LLaMA decode";
  if (!c) return fail(BN_ERR_INVALID_ARG, std::string(op) + ": NULL config");
  if (c->n_layers <= 0 || c->hidden <= 0 || c->n_heads <= 0 || c->n_kv_heads <= 0 ||
      c->intermediate <= 0 || c->vocab <= 0 || c->max_len <= 0)
    return fail(BN_ERR_SHAPE, std::string(op) + ": sizes must be positive");
  if (c->hidden % c->n_heads != 0 || c->hidden / c->n_heads != 64 || c->n_heads % c->n_kv_heads != 0)
    return fail(BN_ERR_UNSUPPORTED,
                std::string(op) + ": head_dim (hidden / n_heads) must be 64 and n_heads a multiple of n_kv_heads");
  if (c->hidden % 4 || c->intermediate % 4 || c->vocab % 4)
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": hidden, intermediate and vocab must be multiples of 4");
  // output-major projections stage their fp32 input row in LDS, padded to
  // whole wave-wide loads (256 elements): refused here, before any launch,
  // rather than by the first projection that cannot stage it
  auto staged = [](int k) { return ((int64_t)k + 255) / 256 * 256; };
  if (c->weights_out_major && (staged(c->hidden) > kGemvStagedMax || staged(c->intermediate) > kGemvStagedMax))
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": output-major weights take hidden and intermediate "
                                                      "sizes of at most " + std::to_string(kGemvStagedMax));
  return BN_OK;
}

}  // namespace
}  // namespace bn

using namespace bn;

extern "C" size_t bn_llama_decode_workspace_size(const bn_llama_config *config) {
  if (check_config(config)) return 0;
  return plan_of(config).total;
}

extern "C" int bn_llama_decode(const bn_llama_config *c, const float *embed, const float *ln_f,
                               const float *lm_head, const bn_llama_layer_weights *layers,
                               int first_token, int position, int n_tokens, uint32_t *tokens_out,
                               void *workspace, size_t workspace_bytes, void *stream) {
  const char *op = "LLaMA decode";
  int st;
  if ((st = check_config(c))) return st;
  if (n_tokens < 0 || position < 0 || (int64_t)position + n_tokens > c->max_len)
    return fail(BN_ERR_SHAPE, std::string(op) + ": position + n_tokens must stay within max_len");
  if (first_token < 0 || first_token >= c->vocab)
    return fail(BN_ERR_INVALID_ARG, std::string(op) + ": first_token outside the vocabulary");
  if (n_tokens == 0) return BN_OK;
  if (!embed || !ln_f || !lm_head || !layers || !tokens_out)
    return fail(BN_ERR_INVALID_ARG, std::string(op) + ": NULL pointer");
  for (int l = 0; l < c->n_layers; ++l) {
    const bn_llama_layer_weights &L = layers[l];
    if (!L.ln1 || !L.wqkv || !L.wo || !L.ln2 || !L.wgu || !L.wd || !L.k_cache || !L.v_cache)
      return fail(BN_ERR_INVALID_ARG, std::string(op) + ": NULL pointer in layer " + std::to_string(l));
  }
  const Plan pl = plan_of(c);
  if (workspace && workspace_bytes < pl.total)
    return fail(BN_ERR_INVALID_ARG, std::string(op) + ": workspace of " + std::to_string(workspace_bytes) +
                                        " bytes, need " + std::to_string(pl.total));
  if (workspace && (reinterpret_cast<uintptr_t>(workspace) & 255u))
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": workspace must be 256-byte aligned");
  if ((st = ensure_device())) return st;
  hipStream_t s = as_stream(stream);
  void *ws = workspace;
  bool own = false;
  if (!ws) {
    if ((st = bn_alloc(&ws, pl.total, stream))) return st;
    own = true;
  }
  char *W = (char *)ws;
  float *hdn = (float *)(W + pl.hdn), *xn = (float *)(W + pl.xn), *qkv = (float *)(W + pl.qkv);
  float *o = (float *)(W + pl.o), *attn = (float *)(W + pl.attn);
  float *act = (float *)(W + pl.act), *mlp = (float *)(W + pl.mlp), *logits = (float *)(W + pl.logits);
  int32_t *lens = (int32_t *)(W + pl.lens);
  void *lin_ws = W + pl.lin, *dec_ws = pl.dec_bytes ? W + pl.dec : nullptr;

  const int hid = c->hidden, hd = 64, kv = c->n_kv_heads * hd, I = c->intermediate;
  const float scale = 0.125f;  // 1 / sqrt(64)
  const bn_view v_hdn = fview(hdn, 1, hid, hid), v_xn = fview(xn, 1, hid, hid);
  const bn_view v_qkv = fview(qkv, 1, hid + 2 * kv, hid + 2 * kv);
  const bn_view v_o = fview(o, 1, hid, hid), v_attn = fview(attn, 1, hid, hid);
  const bn_view v_act = fview(act, 1, I, I), v_mlp = fview(mlp, 1, hid, hid);
  const bn_view v_logits = fview(logits, 1, c->vocab, c->vocab);
  const bool om = c->weights_out_major != 0;
  const bn_view v_lnf = fview(ln_f, 1, hid, hid), v_lm = wview(lm_head, hid, c->vocab, om);

  hipLaunchKernelGGL(fill_lens_kernel, dim3((unsigned)((n_tokens + 255) / 256)), dim3(256), 0, s, lens,
                     position, n_tokens);
  hipError_t e = hipGetLastError();
  st = e == hipSuccess ? BN_OK : hip_fail(e, __FILE__, __LINE__);
  // output-major weights and rows the one-wave norm kernels take: each
  // decode-step RMSNorm (with the residual add before it) is formed in the
  // x staging of the projection that consumes it, and the residual stream
  // alternates between hdn and hdn2 (the projection reads one while its
  // first workgroup writes the other)
  float *const hdn2 = (float *)(W + pl.hdn2);
  const bool fold = om && hid <= kNormRowF32;
  // short caches: the attention's split partials are merged by the O
  // projection (output-major weights)
  const bool merged = om && dec_ws && short_path_ok(BN_F32, 1, c->max_len, c->n_heads);
  for (int t = 0; st == BN_OK && t < n_tokens; ++t) {
    const int pos = position + t;
    hipLaunchKernelGGL(embed_gather_kernel, dim3(1), dim3(256), 0, s, embed,
                       t ? (const uint32_t *)(tokens_out + t - 1) : (const uint32_t *)nullptr,
                       (uint32_t)first_token, c->vocab, hdn, hid,
                       (int)((reinterpret_cast<uintptr_t>(embed) & 15u) == 0));
    if ((e = hipGetLastError()) != hipSuccess) {
      st = hip_fail(e, __FILE__, __LINE__);
      break;
    }
    float *hc = hdn, *hn = hdn2;  // the residual stream now, and the next one
    const bn_view ln10 = fview(layers[0].ln1, 1, hid, hid);
    if (!fold && (st = bn_rmsnorm(&v_hdn, &ln10, &v_xn, c->rms_eps, stream))) break;
    for (int l = 0; l < c->n_layers && st == BN_OK; ++l) {
      const bn_llama_layer_weights &L = layers[l];
      const bn_view wqkv = wview(L.wqkv, hid, hid + 2 * kv, om);
      const bn_view wo = wview(L.wo, hid, hid, om), wgu = wview(L.wgu, hid, 2 * I, om);
      const bn_view wd = wview(L.wd, I, hid, om), ln2 = fview(L.ln2, 1, hid, hid);
      const bn_view nxt = l + 1 < c->n_layers ? fview(layers[l + 1].ln1, 1, hid, hid) : v_lnf;
      // Q, K and V (Q and K rotated at position pos); the epilogue also
      // appends K and V to the caches at row pos.  Folded norms: the input is
      // rmsnorm(h + the previous layer's MLP output) (layer 0: rmsnorm(h))
      const LinNorm n1 = {l ? mlp : nullptr, L.ln1, l ? hn : nullptr, c->rms_eps};
      const bn_view v_hc = fview(hc, 1, hid, hid);
      if ((st = linear_run(fold ? &v_hc : &v_xn, &wqkv, &v_qkv, hid + kv, pos, hd, c->rope_theta, lin_ws,
                           pl.lin_bytes, kLinEpiPlain, L.k_cache + (int64_t)pos * kv,
                           L.v_cache + (int64_t)pos * kv, hid, kv, 0, stream, fold ? &n1 : nullptr)))
        break;
      if (fold && l) std::swap(hc, hn);
      if (merged) {
        // attention as split partials; the O projection merges them in its
        // x staging (the bits of bn_gqa_decode's combine, one launch fewer)
        // (the host knows the length: pos + 1 keys after the append)
        const LinMerge mg = {(const float *)dec_ws, lens + t, kShortSplits, c->max_len, pos + 1};
        if ((st = decode_short_partials(qkv, L.k_cache, L.v_cache, lens + t, pos + 1, (float *)dec_ws, 1,
                                        c->max_len, c->n_heads, c->n_kv_heads, scale, s)))
          break;
        if ((st = linear_run(&v_o, &wo, &v_attn, 0, 0, hd, c->rope_theta, lin_ws, pl.lin_bytes, kLinEpiPlain,
                             nullptr, nullptr, 0, 0, 0, stream, nullptr, &mg)))
          break;
      } else {
        if ((st = bn_gqa_decode(BN_F32, qkv, L.k_cache, L.v_cache, lens + t, o, 1, c->max_len, c->n_heads,
                                c->n_kv_heads, hd, scale, dec_ws, pl.dec_bytes, stream)))
          break;
        if ((st = bn_linear_rope(&v_o, &wo, &v_attn, 0, 0, hd, c->rope_theta, lin_ws, pl.lin_bytes, stream)))
          break;
      }
      // gate | up projection of rmsnorm(h + attention output); its epilogue
      // writes silu(gate) * up
      const LinNorm n2 = {attn, L.ln2, hn, c->rms_eps};
      const bn_view v_hc2 = fview(hc, 1, hid, hid);
      if (!fold && (st = bn_add_rmsnorm(&v_hdn, &v_attn, &ln2, &v_hdn, &v_xn, c->rms_eps, stream))) break;
      if ((st = linear_run(fold ? &v_hc2 : &v_xn, &wgu, &v_act, 0, 0, hd, c->rope_theta, lin_ws, pl.lin_bytes,
                           kLinEpiSilu, nullptr, nullptr, 0, 0, 0, stream, fold ? &n2 : nullptr)))
        break;
      if (fold) std::swap(hc, hn);
      if ((st = bn_linear_rope(&v_act, &wd, &v_mlp, 0, 0, hd, c->rope_theta, lin_ws, pl.lin_bytes, stream)))
        break;
      if (!fold && (st = bn_add_rmsnorm(&v_hdn, &v_mlp, &nxt, &v_hdn, &v_xn, c->rms_eps, stream))) break;
    }
    if (st) break;
    // logits of rmsnorm(h + the last MLP output) * ln_f
    const LinNorm nf = {mlp, ln_f, nullptr, c->rms_eps};
    const bn_view v_hc = fview(hc, 1, hid, hid);
    if ((st = linear_run(fold ? &v_hc : &v_xn, &v_lm, &v_logits, 0, 0, hd, c->rope_theta, lin_ws,
                         pl.lin_bytes, kLinEpiPlain, nullptr, nullptr, 0, 0, 0, stream, fold ? &nf : nullptr)))
      break;
    bn_view tout;
    tout.data = tokens_out + t;
    tout.offset = 0;
    tout.h = 1;
    tout.w = 1;
    tout.stride_h = 1;
    tout.stride_w = 1;
    tout.dtype = BN_U32;
    tout.on_device = 1;
    if ((st = bn_argmax(&v_logits, &tout, stream))) break;
  }
  if (own) {
    const int st2 = bn_free(ws, stream);
    if (st == BN_OK) st = st2;
  }
  return st;
}

// LLaMAModel::embed (llama_model.hpp:161-198) copies the whole table to the
// host, looks the rows up there and copies them back; this gathers on the
// device.
extern "C" int bn_embedding(const bn_view *table, const uint32_t *ids, int n, const bn_view *out,
                            void *stream) {
  const char *op = "embedding";
  const unsigned mask = (1u << BN_F32) | (1u << BN_BF16);
  int st;
  if ((st = check_view(table, op, "table", mask))) return st;
  if ((st = check_view(out, op, "output", mask))) return st;
  if (n < 0) return fail(BN_ERR_SHAPE, std::string(op) + ": negative number of ids");
  if (out->h != n || out->w != table->w)
    return fail(BN_ERR_SHAPE, std::string(op) + ": output must be [n_ids, hidden]");
  if (out->dtype != table->dtype) return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": dtypes differ");
  if ((st = require_device(op, {table, out}))) return st;
  if (n == 0 || out->w == 0) return BN_OK;
  if (!ids) return fail(BN_ERR_INVALID_ARG, std::string(op) + ": NULL ids");
  if ((st = ensure_device())) return st;
  hipStream_t s = as_stream(stream);
  if (table->dtype == BN_F32)
    hipLaunchKernelGGL(embed_rows_kernel<float>, dim3((unsigned)n), dim3(256), 0, s,
                       dview<const float>(table), ids, dview<float>(out));
  else
    hipLaunchKernelGGL(embed_rows_kernel<bf16_t>, dim3((unsigned)n), dim3(256), 0, s,
                       dview<const bf16_t>(table), ids, dview<bf16_t>(out));
  BN_LAUNCH_CHECK();
  return BN_OK;
}
