// extern "C" boundary: argument checks, workspace carving, the Lloyd loop.
//
// Validation mirrors what the reference checks before launching
// (flash_kmeans_cuda/csrc/api.cpp:27-44, assign_sm80.cu:712-731,
// update_sorted.cu:196-206, update_finalize.cu:76-83): shapes, dtypes and
// non-null pointers.  Contiguity is the caller's contract (plain pointers).
// Failures return a status and leave a message in fkc_last_error() instead of
// throwing TORCH_CHECK errors across the ABI.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <atomic>
#include <mutex>
#include <vector>

#include "fkc_internal.hpp"

namespace fkc {

static thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(FKC_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return FKC_OK;
}

static bool env_true(const char* name) {
  const char* s = std::getenv(name);
  return s && (std::strcmp(s, "1") == 0 || std::strcmp(s, "true") == 0);
}

bool force_safe_assign() { return env_true("FKC_ASSIGN_FORCE_SAFE"); }

int ntiles_override() {
  const char* s = std::getenv("FKC_NTILES");
  if (!s) return 0;
  const int v = std::atoi(s);
  return (v == 1 || v == 2 || v == 4 || v == 8) ? v : 0;
}

int ksplit_override() {
  const char* s = std::getenv("FKC_KSPLIT");
  if (!s) return 0;
  const int v = std::atoi(s);
  return (v >= 1 && v <= 64) ? v : 0;
}

int sort_tile_override() {
  const char* s = std::getenv("FKC_SORT_TILE");
  if (!s) return 0;
  const int v = std::atoi(s);
  return (v == 256 || v == 512 || v == 1024 || v == 2048 || v == 4096 ||
          v == 8192) ? v : 0;
}

int save_override() {
  const char* s = std::getenv("FKC_SAVE");
  if (!s || !*s) return -1;
  return std::strcmp(s, "1") == 0 ? 1 : (std::strcmp(s, "0") == 0 ? 0 : -1);
}

int resident_override() {
  const char* s = std::getenv("FKC_RESIDENT");
  if (!s || !*s) return -1;
  return std::strcmp(s, "1") == 0 ? 1 : (std::strcmp(s, "0") == 0 ? 0 : -1);
}

int update_rows_override() {
  const char* s = std::getenv("FKC_UPDATE_ROWS");
  if (!s) return 0;
  const int v = std::atoi(s);
  return (v == 32 || v == 64 || v == 128) ? v : 0;
}

int update_scan_override() {
  const char* s = std::getenv("FKC_UPDATE_SCAN");
  if (!s || !*s) return -1;
  return std::strcmp(s, "1") == 0 ? 1 : (std::strcmp(s, "0") == 0 ? 0 : -1);
}

int scan_wgs_override() {
  const char* s = std::getenv("FKC_SCAN_WGS");
  if (!s) return 0;
  const int v = std::atoi(s);
  return (v >= 1 && v <= 65536) ? v : 0;
}

bool sort_fuse_override() {
  const char* s = std::getenv("FKC_SORT_FUSE");
  return !(s && std::strcmp(s, "0") == 0);
}

int sort_spin_override(int dflt) {
  const char* s = std::getenv("FKC_SORT_SPIN");
  if (!s || !*s) return dflt;
  char* end = nullptr;
  const long v = std::strtol(s, &end, 10);
  return (*end == 0 && v >= 0 && v <= dflt) ? (int)v : dflt;
}

// Device shape, read once per device (the attributes cannot change while
// the process runs); without a usable device (a CPU host asking for
// workspace sizes) the MI355X figures stand in.
DeviceShape device_shape() {
  constexpr int kMaxDev = 64;
  static std::atomic<int> g_cus[kMaxDev];  // 0: not read yet
  static std::atomic<int> g_lds[kMaxDev];
  static std::atomic<bool> g_nodev{false};  // no device: asked once
  DeviceShape d{kMi355xCUs, kMi355xLds};
  int dev = -1;
  if (g_nodev.load(std::memory_order_relaxed)) {
  } else if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) {
    (void)hipGetLastError();  // no device here: do not leave a sticky error
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
      g_nodev.store(true, std::memory_order_relaxed);
    (void)hipGetLastError();
  } else {
    int cus = g_cus[dev].load(std::memory_order_acquire);
    int lds = g_lds[dev].load(std::memory_order_relaxed);
    if (cus == 0) {
      int c = 0, l = 0;
      if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount,
                                dev) != hipSuccess)
        c = 0;
      // LDS one workgroup may use once its kernel opts in (160 KiB on
      // gfx950), else the LDS of a CU.
      if (hipDeviceGetAttribute(&l, hipDeviceAttributeSharedMemPerBlockOptin,
                                dev) != hipSuccess ||
          l <= 0) {
        if (hipDeviceGetAttribute(
                &l, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) !=
            hipSuccess)
          l = 0;
      }
      (void)hipGetLastError();
      cus = c > 0 ? c : kMi355xCUs;
      lds = l > 0 ? l : kMi355xLds;
      g_lds[dev].store(lds, std::memory_order_relaxed);
      g_cus[dev].store(cus, std::memory_order_release);
    }
    d.cus = cus;
    d.lds_per_wg = lds;
  }
  // FKC_CUS=n (tests, A/B runs): plan as if the device had n compute units.
  if (const char* s = std::getenv("FKC_CUS")) {
    char* end = nullptr;
    const long v = std::strtol(s, &end, 10);
    if (*s && *end == 0 && v >= 1 && v <= 4096) d.cus = (int)v;
  }
  return d;
}

// ------------------------------------------------------------- profiling
namespace {
// Process-wide profiling state.  The loop reads `period` without a lock;
// the event lists and totals are only touched under `mu`, so calls from
// several threads are safe (their timed launches are pooled).
struct Profile {
  std::atomic<int> period{0};  // time the assign of every period-th iteration; 0: off
  std::mutex mu;
  std::vector<hipEvent_t> starts, stops;
  double total_ms = 0.0;
  int64_t launches = 0;
};
Profile g_prof;

// Caller holds g_prof.mu.
void prof_clear_events() {
  for (auto e : g_prof.starts) (void)hipEventDestroy(e);
  for (auto e : g_prof.stops) (void)hipEventDestroy(e);
  g_prof.starts.clear();
  g_prof.stops.clear();
}
}  // namespace

static int shape_ok(int64_t B, int64_t N, int64_t K, int64_t D,
                    const char* what) {
  if (B < 0 || N < 0 || K < 1 || D < 1)
    return fail(FKC_ERR_INVALID, "%s: need B>=0, N>=0, K>=1, D>=1 (got %lld %lld %lld %lld)",
                what, (long long)B, (long long)N, (long long)K, (long long)D);
  if (B > 65535 || N > INT32_MAX - 65536 || K > INT32_MAX / 2 ||
      D > (1 << 20))
    return fail(FKC_ERR_UNSUPPORTED, "%s: shape out of supported range", what);
  return FKC_OK;
}

static int dtype_ok(int dtype, const char* what) {
  if (dtype != FKC_F32 && dtype != FKC_F16 && dtype != FKC_BF16)
    return fail(FKC_ERR_INVALID, "%s: unsupported dtype %d", what, dtype);
  return FKC_OK;
}

}  // namespace fkc

// ------------------------------------------------------------- Lloyd loop
namespace fkc {
namespace {
struct LoopBuffers {
  float* x_sq = nullptr;   // only when the VALU assign route is taken
  float* c_sq = nullptr;
  int32_t* sorted = nullptr;
  int32_t* perm = nullptr;
  float* sums = nullptr;
  int32_t* counts = nullptr;
  float* shift = nullptr;  // one slot per iteration
  int32_t* ctrl = nullptr; // [0] converged, [1] iterations run
  void* sort_ws = nullptr;
  size_t sort_ws_bytes = 0;
  void* upd_ws = nullptr;
  size_t upd_ws_bytes = 0;
  void* asg_ws = nullptr;  // sliced assign's partial winners (may be empty)
  size_t asg_ws_bytes = 0;
};

LoopBuffers carve_loop(void* ws, int64_t B, int64_t N, int64_t K, int64_t D,
                       int dtype, int max_iters, size_t* total) {
  Carve c(ws);
  LoopBuffers L;
  if (!assign_uses_mfma(dtype, D)) L.x_sq = c.take<float>((size_t)B * N);
  L.c_sq = c.take<float>((size_t)B * K);
  L.sorted = c.take<int32_t>((size_t)B * N);
  L.perm = c.take<int32_t>((size_t)B * N);
  L.sums = c.take<float>((size_t)B * K * D);
  L.counts = c.take<int32_t>((size_t)B * K);
  L.shift = c.take<float>((size_t)(max_iters > 0 ? max_iters : 1));
  L.ctrl = c.take<int32_t>(4);
  L.sort_ws_bytes = sort_workspace_bytes(B, N, K);
  L.sort_ws = c.take<char>(L.sort_ws_bytes);
  L.upd_ws_bytes = update_workspace_bytes(B, N, D);
  L.upd_ws = c.take<char>(L.upd_ws_bytes);
  L.asg_ws_bytes = assign_workspace_bytes(B, N, K, D, dtype);
  L.asg_ws = L.asg_ws_bytes ? c.take<char>(L.asg_ws_bytes) : nullptr;
  if (total) *total = c.used;
  return L;
}
}  // namespace
}  // namespace fkc

using namespace fkc;

extern "C" {

const char* fkc_last_error(void) { return g_err; }
const char* fkc_version(void) { return "0.1.0"; }

int fkc_euclid_assign(const void* x, const void* centroids, const float* x_sq,
                      const float* c_sq, int32_t* cluster_ids, int64_t B,
                      int64_t N, int64_t K, int64_t D, int dtype,
                      fkc_stream_t stream) {
  g_err[0] = 0;
  if (int rc = shape_ok(B, N, K, D, "euclid_assign")) return rc;
  if (int rc = dtype_ok(dtype, "euclid_assign")) return rc;
  if (B * N == 0) return FKC_OK;
  if (!x || !centroids || !c_sq || !cluster_ids)
    return fail(FKC_ERR_INVALID, "euclid_assign: null pointer argument");
  return launch_assign(x, centroids, x_sq, c_sq, cluster_ids, B, N, K, D, dtype,
                       nullptr, reinterpret_cast<hipStream_t>(stream));
}

size_t fkc_euclid_assign_workspace_bytes(int64_t B, int64_t N, int64_t K,
                                         int64_t D, int dtype) {
  if (shape_ok(B, N, K, D, "euclid_assign_workspace_bytes") ||
      dtype_ok(dtype, "euclid_assign_workspace_bytes"))
    return 0;
  return assign_workspace_bytes(B, N, K, D, dtype);
}

int fkc_euclid_assign_ws(const void* x, const void* centroids,
                         const float* x_sq, const float* c_sq,
                         int32_t* cluster_ids, int64_t B, int64_t N, int64_t K,
                         int64_t D, int dtype, void* workspace,
                         size_t workspace_bytes, fkc_stream_t stream) {
  g_err[0] = 0;
  if (int rc = shape_ok(B, N, K, D, "euclid_assign_ws")) return rc;
  if (int rc = dtype_ok(dtype, "euclid_assign_ws")) return rc;
  if (B * N == 0) return FKC_OK;
  if (!x || !centroids || !c_sq || !cluster_ids)
    return fail(FKC_ERR_INVALID, "euclid_assign_ws: null pointer argument");
  const size_t need = assign_workspace_bytes(B, N, K, D, dtype);
  if (need == 0)
    return launch_assign(x, centroids, x_sq, c_sq, cluster_ids, B, N, K, D,
                         dtype, nullptr, reinterpret_cast<hipStream_t>(stream));
  if (!workspace || workspace_bytes < need)
    return fail(FKC_ERR_WORKSPACE, "euclid_assign_ws: workspace %zu < %zu bytes",
                workspace_bytes, need);
  if (reinterpret_cast<uintptr_t>(workspace) % kWorkspaceAlign != 0)
    return fail(FKC_ERR_WORKSPACE,
                "euclid_assign_ws: workspace not %d-byte aligned",
                kWorkspaceAlign);
  return launch_assign(x, centroids, x_sq, c_sq, cluster_ids, B, N, K, D, dtype,
                       nullptr, reinterpret_cast<hipStream_t>(stream), nullptr,
                       nullptr, workspace, workspace_bytes);
}

int fkc_row_sqnorm(const void* src, float* out, int64_t rows, int64_t D,
                   int dtype, fkc_stream_t stream) {
  g_err[0] = 0;
  if (rows < 0 || D < 1)
    return fail(FKC_ERR_INVALID, "row_sqnorm: need rows>=0, D>=1");
  if (int rc = dtype_ok(dtype, "row_sqnorm")) return rc;
  if (rows == 0) return FKC_OK;
  if (!src || !out) return fail(FKC_ERR_INVALID, "row_sqnorm: null pointer");
  return launch_row_sqnorm(src, out, rows, D, dtype, nullptr,
                           reinterpret_cast<hipStream_t>(stream));
}

size_t fkc_label_sort_workspace_bytes(int64_t B, int64_t N, int64_t K) {
  if (B <= 0 || N <= 0 || K < 1) return 0;
  return sort_workspace_bytes(B, N, K);
}

int fkc_label_sort(const int32_t* cluster_ids, int32_t* sorted_ids,
                   int32_t* perm, int64_t B, int64_t N, int64_t K,
                   void* workspace, size_t workspace_bytes,
                   fkc_stream_t stream) {
  g_err[0] = 0;
  if (int rc = shape_ok(B, N, K, 1, "label_sort")) return rc;
  if (B * N == 0) return FKC_OK;
  if (!cluster_ids || !sorted_ids || !perm)
    return fail(FKC_ERR_INVALID, "label_sort: null pointer argument");
  return launch_label_sort(cluster_ids, sorted_ids, perm, B, N, K, false,
                           workspace, workspace_bytes, nullptr,
                           reinterpret_cast<hipStream_t>(stream));
}

size_t fkc_update_workspace_bytes(int64_t B, int64_t N, int64_t D) {
  if (B <= 0 || N <= 0 || D < 1) return 0;
  return update_workspace_bytes(B, N, D);
}

static int update_common(const void* x, const int32_t* perm,
                         const int32_t* ids_sorted, float* sums,
                         int32_t* counts, int64_t B, int64_t N, int64_t K,
                         int64_t D, int dtype, void* ws, size_t ws_bytes,
                         fkc_stream_t stream, const char* what) {
  g_err[0] = 0;
  if (int rc = shape_ok(B, N, K, D, what)) return rc;
  if (int rc = dtype_ok(dtype, what)) return rc;
  if (B * N == 0) return FKC_OK;
  if (!x || !ids_sorted || !sums || !counts)
    return fail(FKC_ERR_INVALID, "%s: null pointer argument", what);
  return launch_update(x, perm, ids_sorted, sums, counts, B, N, K, D, dtype,
                       false, ws, ws_bytes, nullptr,
                       reinterpret_cast<hipStream_t>(stream));
}

int fkc_centroid_update_sorted(const void* x_sorted, const int32_t* ids_sorted,
                               float* sums, int32_t* counts, int64_t B,
                               int64_t N, int64_t K, int64_t D, int dtype,
                               void* workspace, size_t workspace_bytes,
                               fkc_stream_t stream) {
  return update_common(x_sorted, nullptr, ids_sorted, sums, counts, B, N, K, D,
                       dtype, workspace, workspace_bytes, stream,
                       "centroid_update_sorted");
}

int fkc_centroid_update_sorted_indexed(const void* x, const int32_t* sorted_idx,
                                       const int32_t* ids_sorted, float* sums,
                                       int32_t* counts, int64_t B, int64_t N,
                                       int64_t K, int64_t D, int dtype,
                                       void* workspace, size_t workspace_bytes,
                                       fkc_stream_t stream) {
  if (!sorted_idx && B * N > 0) {
    g_err[0] = 0;
    return fail(FKC_ERR_INVALID,
                "centroid_update_sorted_indexed: null sorted_idx");
  }
  return update_common(x, sorted_idx, ids_sorted, sums, counts, B, N, K, D,
                       dtype, workspace, workspace_bytes, stream,
                       "centroid_update_sorted_indexed");
}

int fkc_centroid_finalize(const float* sums, const int32_t* counts,
                          const void* old_centroids, void* out, int64_t B,
                          int64_t K, int64_t D, int dtype,
                          fkc_stream_t stream) {
  g_err[0] = 0;
  if (int rc = shape_ok(B, 0, K, D, "centroid_finalize")) return rc;
  if (int rc = dtype_ok(dtype, "centroid_finalize")) return rc;
  if (B == 0) return FKC_OK;
  if (!sums || !counts || !old_centroids || !out)
    return fail(FKC_ERR_INVALID, "centroid_finalize: null pointer argument");
  return launch_finalize(sums, counts, old_centroids, out, nullptr, nullptr, B,
                         K, D, dtype, nullptr,
                         reinterpret_cast<hipStream_t>(stream));
}


size_t fkc_quality_workspace_bytes(int64_t B, int64_t N, int64_t K) {
  if (B <= 0 || N < 0 || K < 1) return 0;
  return quality_workspace_bytes(B, N, K);
}

int fkc_assigned_inertia(const void* x, const void* centroids,
                         const int32_t* cluster_ids, int64_t B, int64_t N,
                         int64_t K, int64_t D, int dtype, double* inertia,
                         int32_t* empty_clusters, void* workspace,
                         size_t workspace_bytes, fkc_stream_t stream) {
  g_err[0] = 0;
  if (int rc = shape_ok(B, N, K, D, "assigned_inertia")) return rc;
  if (int rc = dtype_ok(dtype, "assigned_inertia")) return rc;
  if (B == 0 || (!inertia && !empty_clusters)) return FKC_OK;
  if (N > 0 && !cluster_ids)
    return fail(FKC_ERR_INVALID, "assigned_inertia: null cluster_ids");
  if (inertia && N > 0 && (!x || !centroids))
    return fail(FKC_ERR_INVALID,
                "assigned_inertia: x and centroids are needed for inertia");
  return launch_quality(x, centroids, cluster_ids, B, N, K, D, dtype, inertia,
                        empty_clusters, workspace, workspace_bytes,
                        reinterpret_cast<hipStream_t>(stream));
}

size_t fkc_sampled_inertia_workspace_bytes(int64_t B, int64_t S, int64_t K,
                                           int64_t D, int dtype) {
  if (B <= 0 || S <= 0 || K < 1 || D < 1 || dtype_ok(dtype, "sampled_inertia"))
    return 0;
  return sample_workspace_bytes(B, S, K, D, dtype);
}

int fkc_sampled_inertia(const void* x, const void* centroids,
                        const int32_t* sample_idx, int64_t S, int64_t B,
                        int64_t N, int64_t K, int64_t D, int dtype,
                        double* inertia, void* workspace,
                        size_t workspace_bytes, fkc_stream_t stream) {
  g_err[0] = 0;
  if (int rc = shape_ok(B, N, K, D, "sampled_inertia")) return rc;
  if (int rc = dtype_ok(dtype, "sampled_inertia")) return rc;
  if (S < 0 || S > INT32_MAX - 65536)
    return fail(FKC_ERR_INVALID, "sampled_inertia: bad sample count %lld",
                (long long)S);
  if (B == 0) return FKC_OK;
  if (!inertia) return fail(FKC_ERR_INVALID, "sampled_inertia: null inertia");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (S == 0 || N == 0) return launch_fill_f64(inertia, 0.0, B, s);
  if (!x || !centroids || !sample_idx)
    return fail(FKC_ERR_INVALID, "sampled_inertia: null pointer argument");
  return launch_sampled_inertia(x, centroids, sample_idx, S, B, N, K, D, dtype,
                                inertia, workspace, workspace_bytes, s);
}

size_t fkc_kmeans_workspace_bytes(int64_t B, int64_t N, int64_t K, int64_t D,
                                  int dtype, int max_iters) {
  if (B <= 0 || N <= 0 || K < 1 || D < 1) return 256;
  size_t total = 0;
  carve_loop(nullptr, B, N, K, D, dtype, max_iters, &total);
  return total;
}

size_t fkc_kmeans_sort_recounts_offset(int64_t B, int64_t N, int64_t K,
                                       int64_t D, int dtype, int max_iters) {
  if (B <= 0 || N <= 0 || K < 1 || D < 1) return 0;
  // The recount word is the first int32 of the sort's control region, which
  // the loop's prologue clears; carving from a non-null base at 0 gives the
  // offsets (the base is never dereferenced).
  char* const base = reinterpret_cast<char*>(kWorkspaceAlign);
  const LoopBuffers L = carve_loop(base, B, N, K, D, dtype, max_iters, nullptr);
  int32_t* p = nullptr;
  int64_t n = 0;
  label_sort_reset_region(L.sort_ws, B, N, K, &p, &n);
  return n > 0 ? (size_t)(reinterpret_cast<char*>(p) - base) : 0;
}

}  // extern "C"

namespace fkc {
// fkc_kmeans_lloyd (init == centroids), fkc_kmeans_lloyd_from and the
// static-scratch fkc_kmeans_lloyd_noalloc (profile = false: no events).
int lloyd_run(const void* x, const void* init, void* centroids,
              int32_t* cluster_ids, int64_t B, int64_t N, int64_t K,
              int64_t D, int dtype, int max_iters, float tol, void* workspace,
              size_t workspace_bytes, fkc_stream_t stream,
              int32_t* n_iters_dev, int32_t* n_iters_host, bool profile) {
  g_err[0] = 0;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (int rc = shape_ok(B, N, K, D, "kmeans_lloyd")) return rc;
  if (int rc = dtype_ok(dtype, "kmeans_lloyd")) return rc;
  if (max_iters < 0) return fail(FKC_ERR_INVALID, "kmeans_lloyd: max_iters < 0");
  if (B == 0 || N == 0 || max_iters == 0) {
    if (n_iters_host) *n_iters_host = (B == 0 || N == 0) ? max_iters : 0;
    // The centroids returned are the initial ones.
    if (B > 0 && init != centroids) {
      if (!init || !centroids)
        return fail(FKC_ERR_INVALID, "kmeans_lloyd: null pointer argument");
      const size_t esz = dtype == FKC_F32 ? 4 : 2;
      if (hipMemcpyAsync(centroids, init, (size_t)B * K * D * esz,
                         hipMemcpyDeviceToDevice, s) != hipSuccess)
        return fail(FKC_ERR_LAUNCH, "kmeans_lloyd: copy of the initial centroids failed");
    }
    if (n_iters_dev)
      return launch_fill_i32(n_iters_dev, (B == 0 || N == 0) ? max_iters : 0,
                             1, s);
    return FKC_OK;
  }
  if (!x || !init || !centroids || !cluster_ids)
    return fail(FKC_ERR_INVALID, "kmeans_lloyd: null pointer argument");
  size_t need = 0;
  carve_loop(nullptr, B, N, K, D, dtype, max_iters, &need);
  if (!workspace || workspace_bytes < need)
    return fail(FKC_ERR_WORKSPACE, "kmeans_lloyd: workspace %zu < %zu bytes",
                workspace_bytes, need);
  if (reinterpret_cast<uintptr_t>(workspace) % kWorkspaceAlign != 0)
    return fail(FKC_ERR_WORKSPACE, "kmeans_lloyd: workspace not %d-byte aligned",
                kWorkspaceAlign);
  LoopBuffers L = carve_loop(workspace, B, N, K, D, dtype, max_iters, nullptr);

  const bool check = tol > 0.f;
  const int32_t* ctrl = check ? L.ctrl : nullptr;
  const bool scan = update_scan_ok(B, N, K, D);
  // One prologue launch: copy of the initial centroids (when separate),
  // their c_sq, and the zeroing of the control words, the sort's and the
  // update's control regions and the shift slots.
  ZeroFill zf;
  zf.z0 = L.ctrl;
  zf.n0 = 4;
  label_sort_reset_region(L.sort_ws, B, N, K, &zf.z1, &zf.n1);
  update_control_region(L.upd_ws, B, N, D, &zf.z3, &zf.n3);
  if (check) {
    zf.z2 = L.shift;
    zf.n2 = max_iters;
  }
  int rc = launch_lloyd_prologue(init, centroids, L.c_sq, B * K, D, dtype, zf, s);
  if (!rc && L.x_sq) rc = launch_row_sqnorm(x, L.x_sq, B * N, D, dtype, nullptr, s);
  if (rc) return rc;

  for (int it = 0; it < max_iters; ++it) {
    // Profiling: the assign's dispatch stamps the two events.  They only
    // carry timestamps, so they skip the system-scope fence (cache write-back
    // and invalidate) an event otherwise implies, which cost ~5 us around
    // each assign.
    hipEvent_t e0 = nullptr, e1 = nullptr;
    const int period =
        profile ? g_prof.period.load(std::memory_order_relaxed) : 0;
    // The middle iteration of each run of `period` (k/2, k/2 + k, ...):
    // with a clock that still drifts over the first iterations, midpoints
    // estimate the mean launch time without the bias of always sampling a
    // run's first iteration.
    if (period > 0 && it % period == period / 2) {
      if (hipEventCreateWithFlags(&e0, hipEventDisableSystemFence) != hipSuccess)
        return fail(FKC_ERR_LAUNCH, "kmeans_lloyd: profiling event creation failed");
      if (hipEventCreateWithFlags(&e1, hipEventDisableSystemFence) != hipSuccess) {
        (void)hipEventDestroy(e0);
        return fail(FKC_ERR_LAUNCH, "kmeans_lloyd: profiling event creation failed");
      }
    }
    rc = launch_assign(x, centroids, L.x_sq, L.c_sq, cluster_ids, B, N, K, D,
                       dtype, ctrl, s, e0, e1, L.asg_ws, L.asg_ws_bytes);
    // The events join the shared lists only once recorded, so another
    // thread's fkc_profile_enable cannot destroy them before that.
    if (e0 != nullptr) {
      if (rc) {
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
      } else {
        std::lock_guard<std::mutex> lock(g_prof.mu);
        g_prof.starts.push_back(e0);
        g_prof.stops.push_back(e1);
      }
    }
    // The update finalizes the centroids itself when D <= 512 (no sums /
    // counts round trip); otherwise finalize runs as its own kernel.  Short
    // rows take the sort-free update: one launch, the same bits.
    const UpdateFinalize fin{centroids, L.c_sq, check ? L.shift + it : nullptr};
    bool fused = false;
    if (!rc && scan) {
      rc = launch_update_scan(x, cluster_ids, B, N, K, D, dtype, L.upd_ws,
                              L.upd_ws_bytes, ctrl, s, fin);
      fused = true;
    }
    if (!rc && !scan)
      rc = launch_label_sort(cluster_ids, L.sorted, L.perm, B, N, K, true,
                             L.sort_ws, L.sort_ws_bytes, ctrl, s, it);
    if (!rc && !scan)
      rc = launch_update(x, L.perm, L.sorted, L.sums, L.counts, B, N, K, D,
                         dtype, true, L.upd_ws, L.upd_ws_bytes, ctrl, s, &fin,
                         &fused, it);
    if (!rc && !fused)
      rc = launch_finalize(L.sums, L.counts, centroids, centroids, L.c_sq,
                           check ? L.shift + it : nullptr, B, K, D, dtype, ctrl,
                           s);
    if (!rc && check) rc = launch_converge_check(L.shift, it, tol, L.ctrl, s);
    if (rc) return rc;
  }
  if (!check && n_iters_dev) rc = launch_fill_i32(n_iters_dev, max_iters, 1, s);
  if (check && n_iters_dev) {
    if (hipMemcpyAsync(n_iters_dev, L.ctrl + 1, sizeof(int32_t),
                       hipMemcpyDeviceToDevice, s) != hipSuccess)
      return fail(FKC_ERR_LAUNCH, "kmeans_lloyd: copy of iteration count failed");
  }
  if (rc) return rc;
  if (n_iters_host) {
    if (!check) {
      *n_iters_host = max_iters;
    } else {
      int32_t v = 0;
      if (hipMemcpyAsync(&v, L.ctrl + 1, sizeof(int32_t), hipMemcpyDeviceToHost,
                         s) != hipSuccess ||
          hipStreamSynchronize(s) != hipSuccess)
        return fail(FKC_ERR_LAUNCH, "kmeans_lloyd: reading iteration count failed");
      *n_iters_host = v;
    }
  }
  return FKC_OK;
}
}  // namespace fkc

extern "C" {

int fkc_kmeans_lloyd(const void* x, void* centroids, int32_t* cluster_ids,
                     int64_t B, int64_t N, int64_t K, int64_t D, int dtype,
                     int max_iters, float tol, void* workspace,
                     size_t workspace_bytes, fkc_stream_t stream,
                     int32_t* n_iters_dev, int32_t* n_iters_host) {
  return lloyd_run(x, centroids, centroids, cluster_ids, B, N, K, D, dtype,
                   max_iters, tol, workspace, workspace_bytes, stream,
                   n_iters_dev, n_iters_host, true);
}

int fkc_kmeans_lloyd_from(const void* x, const void* init_centroids,
                          void* centroids, int32_t* cluster_ids, int64_t B,
                          int64_t N, int64_t K, int64_t D, int dtype,
                          int max_iters, float tol, void* workspace,
                          size_t workspace_bytes, fkc_stream_t stream,
                          int32_t* n_iters_dev, int32_t* n_iters_host) {
  return lloyd_run(x, init_centroids, centroids, cluster_ids, B, N, K, D,
                   dtype, max_iters, tol, workspace, workspace_bytes, stream,
                   n_iters_dev, n_iters_host, true);
}

void fkc_profile_enable(int enable) {
  std::lock_guard<std::mutex> lock(g_prof.mu);
  g_prof.period.store(enable > 0 ? enable : 0, std::memory_order_relaxed);
  prof_clear_events();
  g_prof.total_ms = 0.0;
  g_prof.launches = 0;
}

int fkc_profile_assign_ms(double* total_ms, int64_t* launches) {
  std::lock_guard<std::mutex> lock(g_prof.mu);
  double tot = 0.0;
  for (size_t i = 0; i < g_prof.starts.size(); ++i) {
    if (hipEventSynchronize(g_prof.stops[i]) != hipSuccess)
      return fail(FKC_ERR_LAUNCH, "profile: event sync failed");
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, g_prof.starts[i], g_prof.stops[i]) != hipSuccess)
      return fail(FKC_ERR_LAUNCH, "profile: elapsed time failed");
    tot += ms;
  }
  g_prof.total_ms += tot;
  g_prof.launches += (int64_t)g_prof.starts.size();
  prof_clear_events();
  if (total_ms) *total_ms = g_prof.total_ms;
  if (launches) *launches = g_prof.launches;
  return FKC_OK;
}

}  // extern "C"
