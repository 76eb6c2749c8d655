// bn_runtime.hip -- runtime half of the C ABI: error reporting, device and
// stream handling, the stream-ordered memory pool and host<->device copies.
//
// The pool replaces the reference's CudaMemoryPool (src/utils/memory_pool.cuh:
// 15-125, never used there) and the per-tensor cudaMalloc/cudaFree of
// Tensor<T> (src/utils/tensor.cuh:15-26, 59-77), whose cudaFree synchronised
// the device on every temporary.  Here every allocation is a hipMallocAsync
// on the device's default memory pool with its release threshold raised to
// "never", so freed blocks stay cached in the driver pool and a free is a
// stream-ordered hipFreeAsync: no device synchronisation on the hot path.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <unordered_map>

#include "bn_common.hpp"

namespace bn {

static thread_local std::string t_last_error;

void set_error(const std::string &msg) { t_last_error = msg; }

int hip_fail(hipError_t err, const char *file, int line) {
  const char *base = std::strrchr(file, '/');
  set_error(std::string("HIP Error: ") + hipGetErrorString(err) + " (" +
            std::to_string((int)err) + ") at " + (base ? base + 1 : file) + ":" +
            std::to_string(line));
  return BN_ERR_HIP;
}

// ------------------------------------------------------------------ device
static std::mutex g_mu;
static int g_device = -1;          // device chosen by bn_init (lazily 0)
static hipMemPool_t g_pool = nullptr;
static thread_local int t_device = -1;

static int init_locked(int device) {
  int n = 0;
  BN_HIP_TRY(hipGetDeviceCount(&n));
  if (device < 0 || device >= n)
    return fail(BN_ERR_INVALID_ARG, "bn_init: device " + std::to_string(device) +
                                        " out of range (" + std::to_string(n) + " devices)");
  BN_HIP_TRY(hipSetDevice(device));
  // the no-allocation decode entry point's scratch array: its address on
  // this device, looked up once while the device is current
  int st = decode_scratch_setup(device);
  if (st != BN_OK) return st;
  hipMemPool_t pool = nullptr;
  BN_HIP_TRY(hipDeviceGetDefaultMemPool(&pool, device));
  uint64_t threshold = UINT64_MAX;  // keep freed memory cached in the pool
  BN_HIP_TRY(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &threshold));
  g_device = device;
  g_pool = pool;
  t_device = device;
  return BN_OK;
}

int ensure_device() {
  if (g_device < 0) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_device < 0) {
      int st = init_locked(0);
      if (st != BN_OK) return st;
    }
  }
  if (t_device != g_device) {
    BN_HIP_TRY(hipSetDevice(g_device));
    t_device = g_device;
  }
  return BN_OK;
}

int library_device() { return g_device; }

int device_cu_count() {
  static int cached_device = -1, cached_count = 0;
  std::lock_guard<std::mutex> lk(g_mu);
  if (cached_device != g_device) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, g_device) != hipSuccess)
      n = 0;
    cached_device = g_device;
    cached_count = n;
  }
  return cached_count;
}

// -------------------------------------------------------------- validation
int check_view(const bn_view *v, const char *op, const char *name, unsigned dtype_mask,
               bool need_device) {
  std::string who = std::string(op) + ": " + name;
  if (!v) return fail(BN_ERR_INVALID_ARG, who + " view is NULL");
  if (v->h < 0 || v->w < 0) return fail(BN_ERR_SHAPE, who + " has a negative dimension");
  if (v->dtype < 0 || v->dtype > BN_U32 || !((dtype_mask >> v->dtype) & 1u))
    return fail(BN_ERR_UNSUPPORTED, who + " has an unsupported dtype");
  if (need_device && !v->on_device)
    return fail(BN_ERR_NOT_DEVICE, std::string(op) + ": only GPU implementation available");
  if (!v->data && (int64_t)v->h * v->w > 0)
    return fail(BN_ERR_INVALID_ARG, who + " has a NULL data pointer");
  if (v->offset < 0) return fail(BN_ERR_INVALID_ARG, who + " has a negative offset");
  return BN_OK;
}

int make_rope_freqs(const char *op, int head_dim, float theta, RopeFreqs *out) {
  if (head_dim <= 0 || head_dim % 2 != 0)
    return fail(BN_ERR_SHAPE, std::string(op) + ": head_dim must be a positive even number");
  if (head_dim / 2 > kMaxRopePairs)
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": head_dim above " +
                                        std::to_string(2 * kMaxRopePairs) + " is not supported");
  for (int p = 0; p < head_dim / 2; ++p) {
    // op_rope.cuh:82: exponent in fp32, theta^e in fp32, reciprocal in double
    float e = (float)(2 * p) / (float)head_dim;
    float tp = (float)std::pow((double)theta, (double)e);
    out->f[p] = (float)(1.0 / (double)tp);
  }
  return BN_OK;
}

// -------------------------------------------------------------------- pool
struct PoolState {
  std::mutex mu;
  std::unordered_map<void *, size_t> live;
  uint64_t in_use = 0, peak = 0, n_alloc = 0, n_free = 0;
  size_t limit = 0;
};
static PoolState &pool_state() {
  static PoolState *s = new PoolState();  // never destroyed: frees may run at exit
  return *s;
}

}  // namespace bn

using namespace bn;

extern "C" {

int bn_abi_version(void) { return BN_ABI_VERSION; }

const char *bn_last_error(void) { return t_last_error.c_str(); }

int bn_init(int device) {
  std::lock_guard<std::mutex> lk(g_mu);
  return init_locked(device);
}

int bn_device_count(int *count) {
  if (!count) return fail(BN_ERR_INVALID_ARG, "bn_device_count: NULL output");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e == hipErrorNoDevice) n = 0;
  else if (e != hipSuccess) return hip_fail(e, __FILE__, __LINE__);
  *count = n;
  return BN_OK;
}

int bn_stream_create(void **stream) {
  if (!stream) return fail(BN_ERR_INVALID_ARG, "bn_stream_create: NULL output");
  int st = ensure_device();
  if (st) return st;
  hipStream_t s;
  BN_HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = s;
  return BN_OK;
}

int bn_stream_destroy(void *stream) {
  if (!stream) return BN_OK;
  BN_HIP_TRY(hipStreamDestroy(as_stream(stream)));
  return BN_OK;
}

int bn_stream_synchronize(void *stream) {
  int st = ensure_device();
  if (st) return st;
  BN_HIP_TRY(hipStreamSynchronize(as_stream(stream)));
  return BN_OK;
}

int bn_device_synchronize(void) {
  int st = ensure_device();
  if (st) return st;
  BN_HIP_TRY(hipDeviceSynchronize());
  return BN_OK;
}

int bn_mem_get_info(size_t *free_bytes, size_t *total_bytes) {
  if (!free_bytes || !total_bytes) return fail(BN_ERR_INVALID_ARG, "bn_mem_get_info: NULL output");
  int st = ensure_device();
  if (st) return st;
  BN_HIP_TRY(hipMemGetInfo(free_bytes, total_bytes));
  return BN_OK;
}

int bn_alloc(void **ptr, size_t bytes, void *stream) {
  if (!ptr) return fail(BN_ERR_INVALID_ARG, "bn_alloc: NULL output pointer");
  *ptr = nullptr;
  if (bytes == 0) return BN_OK;
  int st = ensure_device();
  if (st) return st;
  PoolState &ps = pool_state();
  {
    std::lock_guard<std::mutex> lk(ps.mu);
    if (ps.limit && ps.in_use + bytes > ps.limit)
      return fail(BN_ERR_OOM, "bn_alloc: pool limit of " + std::to_string(ps.limit) +
                                  " bytes exceeded by a request of " + std::to_string(bytes));
  }
  void *p = nullptr;
  hipError_t e = hipMallocAsync(&p, bytes, as_stream(stream));
  if (e == hipErrorOutOfMemory) {
    (void)hipGetLastError();
    return fail(BN_ERR_OOM, "bn_alloc: out of device memory for " + std::to_string(bytes) +
                                " bytes");
  }
  if (e != hipSuccess) return hip_fail(e, __FILE__, __LINE__);
  std::lock_guard<std::mutex> lk(ps.mu);
  ps.live[p] = bytes;
  ps.in_use += bytes;
  if (ps.in_use > ps.peak) ps.peak = ps.in_use;
  ps.n_alloc++;
  *ptr = p;
  return BN_OK;
}

int bn_free(void *ptr, void *stream) {
  if (!ptr) return BN_OK;
  PoolState &ps = pool_state();
  size_t bytes = 0;
  {
    std::lock_guard<std::mutex> lk(ps.mu);
    auto it = ps.live.find(ptr);
    if (it == ps.live.end())
      return fail(BN_ERR_INVALID_ARG, "bn_free: pointer was not allocated by bn_alloc");
    bytes = it->second;
    ps.live.erase(it);
    ps.in_use -= bytes;
    ps.n_free++;
  }
  int st = ensure_device();
  if (st) return st;
  BN_HIP_TRY(hipFreeAsync(ptr, as_stream(stream)));
  return BN_OK;
}

int bn_pool_get_stats(bn_pool_stats *out) {
  if (!out) return fail(BN_ERR_INVALID_ARG, "bn_pool_get_stats: NULL output");
  PoolState &ps = pool_state();
  {
    std::lock_guard<std::mutex> lk(ps.mu);
    out->bytes_in_use = ps.in_use;
    out->peak_bytes_in_use = ps.peak;
    out->n_allocs = ps.n_alloc;
    out->n_frees = ps.n_free;
    out->n_live = ps.live.size();
  }
  out->bytes_reserved = 0;
  if (g_pool) {
    uint64_t r = 0;
    if (hipMemPoolGetAttribute(g_pool, hipMemPoolAttrReservedMemCurrent, &r) == hipSuccess)
      out->bytes_reserved = r;
  }
  return BN_OK;
}

int bn_pool_reset_peak(void) {
  PoolState &ps = pool_state();
  std::lock_guard<std::mutex> lk(ps.mu);
  ps.peak = ps.in_use;
  return BN_OK;
}

int bn_pool_trim(size_t min_bytes_to_keep) {
  int st = ensure_device();
  if (st) return st;
  BN_HIP_TRY(hipDeviceSynchronize());
  BN_HIP_TRY(hipMemPoolTrimTo(g_pool, min_bytes_to_keep));
  return BN_OK;
}

int bn_pool_set_limit(size_t limit_bytes) {
  PoolState &ps = pool_state();
  std::lock_guard<std::mutex> lk(ps.mu);
  ps.limit = limit_bytes;
  return BN_OK;
}

int bn_memcpy(void *dst, const void *src, size_t bytes, int kind, void *stream) {
  if (bytes == 0) return BN_OK;
  if (!dst || !src) return fail(BN_ERR_INVALID_ARG, "bn_memcpy: NULL pointer");
  if (kind == 3) {
    std::memcpy(dst, src, bytes);
    return BN_OK;
  }
  hipMemcpyKind k;
  switch (kind) {
    case 0: k = hipMemcpyHostToDevice; break;
    case 1: k = hipMemcpyDeviceToHost; break;
    case 2: k = hipMemcpyDeviceToDevice; break;
    default: return fail(BN_ERR_INVALID_ARG, "bn_memcpy: kind must be 0..3");
  }
  int st = ensure_device();
  if (st) return st;
  hipStream_t s = as_stream(stream);
  BN_HIP_TRY(hipMemcpyAsync(dst, src, bytes, k, s));
  if (kind != 2) BN_HIP_TRY(hipStreamSynchronize(s));
  return BN_OK;
}

}  // extern "C"
