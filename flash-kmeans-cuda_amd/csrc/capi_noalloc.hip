// fkc_kmeans_lloyd_noalloc: the Lloyd loop with its workspace in a static
// device array, for callers that cannot allocate device memory (code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// The array, `scratch`, is a file-scope __device__ variable of
// kScratchBytes: every GPU that loads this library holds one copy of it
// until the process ends.  In host code the name `scratch` stands for a
// host-side shadow, not a device address, so the device address is looked
// up once per device with hipGetSymbolAddress (on the first call made with
// that device current) and only that pointer is ever handed to kernels.
//
// The loop reuses the array across calls: everything the loop needs zeroed
// is cleared by its own prologue kernel, so stale contents from an earlier
// call do not matter, but two calls that overlap on one GPU (different
// streams, or different host threads) share the array and race.  No call
// here allocates, frees, or creates events.
#include <hip/hip_runtime.h>

#include <mutex>

#include "fkc_internal.hpp"

namespace fkc {
namespace {

constexpr size_t kScratchBytes = size_t(64) << 20;  // 64 MiB per GPU
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up once).
int scratch_on_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess)
    return fail(FKC_ERR_LAUNCH, "kmeans_lloyd_noalloc: no current HIP device");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(FKC_ERR_UNSUPPORTED, "kmeans_lloyd_noalloc: device %d >= %d", dev,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(FKC_ERR_LAUNCH,
                  "kmeans_lloyd_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FKC_OK;
}

}  // namespace
}  // namespace fkc

extern "C" {

size_t fkc_kmeans_noalloc_max_bytes(void) { return fkc::kScratchBytes; }

int fkc_kmeans_lloyd_noalloc(const void* x, const void* init_centroids,
                             void* centroids, int32_t* cluster_ids, int64_t B,
                             int64_t N, int64_t K, int64_t D, int dtype,
                             int max_iters, float tol, fkc_stream_t stream,
                             int32_t* n_iters_dev, int32_t* n_iters_host) {
  const size_t need =
      fkc_kmeans_workspace_bytes(B, N, K, D, dtype, max_iters < 0 ? 0 : max_iters);
  if (need > fkc::kScratchBytes)
    return fkc::fail(FKC_ERR_WORKSPACE,
                     "kmeans_lloyd_noalloc: this shape needs %zu bytes of "
                     "workspace; the static scratch holds %zu",
                     need, fkc::kScratchBytes);
  void* ws = nullptr;
  if (int rc = fkc::scratch_on_current_device(&ws)) return rc;
  return fkc::lloyd_run(x, init_centroids, centroids, cluster_ids, B, N, K, D,
                        dtype, max_iters, tol, ws, fkc::kScratchBytes, stream,
                        n_iters_dev, n_iters_host, /*profile=*/false);
}

}  // extern "C"
