// Internal declarations shared by the gfx950 kernels and the C ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "fkc.h"

namespace fkc {

// ---------------------------------------------------------------- errors
// Record a printf-style message as this thread's last error; returns `code`.
int fail(int code, const char* fmt, ...);
// Map the sticky launch status after a kernel launch to an FKC status.
int check_launch(const char* what);

// ---------------------------------------------------------------- sizes
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
inline size_t dtype_size(int dtype) { return dtype == FKC_F32 ? 4 : 2; }

// Bump allocator over a caller-owned workspace.
// Workspaces are carved in 256-byte aligned slices and read with 16-byte
// vector loads, so their base must be 256-byte aligned (hipMalloc and the
// torch caching allocator return such pointers).
constexpr int kWorkspaceAlign = 256;

struct Carve {
  char* base;
  size_t used = 0;
  explicit Carve(void* p) : base(static_cast<char*>(p)) {}
  template <typename T>
  T* take(size_t count) {
    size_t off = used;
    used = align_up(used + count * sizeof(T), 256);
    return base ? reinterpret_cast<T*>(base + off) : nullptr;
  }
};

// ---------------------------------------------------------------- assign
// Routing predicate: the MFMA kernel serves fp16/bf16, D % 8 == 0, D <= 512.
bool assign_uses_mfma(int dtype, int64_t D);
// Workspace bytes of a sliced MFMA assign (centroid slices scored by
// separate workgroups, then merged) for this shape; 0 when it is not sliced.
size_t assign_workspace_bytes(int64_t B, int64_t N, int64_t K, int64_t D,
                              int dtype);
// ev0 / ev1 (optional, both or neither): timing events of the launch; on
// the MFMA route the dispatch packets stamp them (no extra stream packets).
// ws (optional, assign_workspace_bytes): with it the MFMA route may slice K;
// without it the launch is never sliced.
int launch_assign(const void* x, const void* c, const float* x_sq,
                  const float* c_sq, int32_t* ids, int64_t B, int64_t N,
                  int64_t K, int64_t D, int dtype, const int32_t* ctrl,
                  hipStream_t s, hipEvent_t ev0 = nullptr,
                  hipEvent_t ev1 = nullptr, void* ws = nullptr,
                  size_t ws_bytes = 0);
int launch_row_sqnorm(const void* src, float* out, int64_t rows, int64_t D,
                      int dtype, const int32_t* ctrl, hipStream_t s);

// ---------------------------------------------------------------- sort
struct SortPlan {
  int passes = 0;       // LSD passes (0 when K == 1)
  int bits[4] = {0};    // digit width of each pass
  int shift[4] = {0};   // bit offset of each pass
  int64_t ntiles = 0;   // key tiles per batch row
  int tile = 4096;      // keys per tile
};
// labels_valid: the caller guarantees every label is in [0,K), which saves
// the sentinel bin (K = 256 then sorts in one 8-bit pass).
SortPlan sort_plan(int64_t B, int64_t N, int64_t K, bool labels_valid);
size_t sort_workspace_bytes(int64_t B, int64_t N, int64_t K);
// Tiles of this size one launch may hold that all run at once on the
// current device (CUs x workgroups per CU, capped): grids within it chain
// by block index and count their digits in the first pass.
int64_t sort_resident_tiles(int tile);
// seq < 0: standalone call (clears the workspace's control region first).
// seq >= 0: the number of earlier calls on this workspace since the caller
// cleared it with label_sort_reset (0, 1, 2, ... over consecutive calls of
// one shape, each enqueued after the previous one).
int launch_label_sort(const int32_t* ids, int32_t* sorted_ids, int32_t* perm,
                      int64_t B, int64_t N, int64_t K, bool labels_valid,
                      void* ws, size_t ws_bytes, const int32_t* ctrl,
                      hipStream_t s, int64_t seq = -1);
int label_sort_reset(void* ws, int64_t B, int64_t N, int64_t K, hipStream_t s);
// The int32 region label_sort_reset zeroes (for fusing it into another
// launch): *p, *n (n = 0 when B * N == 0).
void label_sort_reset_region(void* ws, int64_t B, int64_t N, int64_t K,
                             int32_t** p, int64_t* n);
// FKC_SORT_TILE=256|512|1024|2048|4096|8192: keys per sort tile; 0 = auto.
int sort_tile_override();
// FKC_SORT_SPIN=n (n >= 0, tests): spin budget of the sort's waits instead
// of dflt; 0 sends every wait (look-back walk, row barrier) to its recount.
int sort_spin_override(int dflt);
// FKC_SORT_FUSE=0: count digits in a separate upsweep also where the first
// pass could count them itself (false); otherwise true.
bool sort_fuse_override();

// ---------------------------------------------------------------- update
size_t update_workspace_bytes(int64_t B, int64_t N, int64_t D);
// overwrite=false: sums/counts += run totals (caller zeroed them).
// overwrite=true : every bin of sums/counts is written (absent bins get 0);
//                  requires every label in [0,K) and sorted order.
// Finalize fused into the update (Lloyd loop, overwrite mode): the new
// centroids are written in place to `cent`, their squared norms to `c_sq`,
// the max shift to `shift` (may be null), so no sums/counts round trip and
// no finalize launch are needed.
struct UpdateFinalize {
  void* cent;
  float* c_sq;
  float* shift;
};
// fin: optional fused finalize; *fused (may be null) reports whether it was
// applied (it needs D <= 512); when not, the caller runs launch_finalize.
// seq >= 0 (overwrite mode only): the number of earlier calls on this
// workspace since the caller cleared its control region
// (update_control_region), over consecutive calls of one shape, each
// enqueued after the previous one; block partials are then computed inside
// the run kernel.  seq < 0: standalone.
int launch_update(const void* x, const int32_t* perm /*nullable*/,
                  const int32_t* ids_sorted, float* sums, int32_t* counts,
                  int64_t B, int64_t N, int64_t K, int64_t D, int dtype,
                  bool overwrite, void* ws, size_t ws_bytes,
                  const int32_t* ctrl, hipStream_t s,
                  const UpdateFinalize* fin = nullptr, bool* fused = nullptr,
                  int64_t seq = -1);
// Sort-free update of the Lloyd loop (no label sort, one launch) for short
// rows: whether the plan takes it for this shape (FKC_UPDATE_SCAN=0|1 turns
// it off / on where it can run), and its launch.  Overwrite mode with the
// finalize fused, every label in [0,K); `ws` is an update workspace
// (update_workspace_bytes); the centroids, c_sq and shift equal those of
// launch_label_sort + launch_update bit for bit.
bool update_scan_ok(int64_t B, int64_t N, int64_t K, int64_t D);
int launch_update_scan(const void* x, const int32_t* ids, int64_t B,
                       int64_t N, int64_t K, int64_t D, int dtype, void* ws,
                       size_t ws_bytes, const int32_t* ctrl, hipStream_t s,
                       const UpdateFinalize& fin);
// The int32 region of an update workspace that a sequenced caller zeroes
// before its first call: *p, *n (n = 0 when B * N == 0).
void update_control_region(void* ws, int64_t B, int64_t N, int64_t D,
                           int32_t** p, int64_t* n);

// ---------------------------------------------------------------- finalize
// c_sq_out / shift_out may be null.  shift_out receives max over rows of
// ||new-old||_2 through an atomic max (caller zeroes it).
int launch_finalize(const float* sums, const int32_t* counts, const void* old,
                    void* out, float* c_sq_out, float* shift_out, int64_t B,
                    int64_t K, int64_t D, int dtype, const int32_t* ctrl,
                    hipStream_t s);

// ---------------------------------------------------------------- misc
int launch_fill_i32(int32_t* p, int32_t v, int64_t n, hipStream_t s);
// Zero-fills fused into the Lloyd prologue (null pointer / zero count: none).
struct ZeroFill {
  int32_t* z0 = nullptr;
  int64_t n0 = 0;
  int32_t* z1 = nullptr;
  int64_t n1 = 0;
  float* z2 = nullptr;
  int64_t n2 = 0;
  int32_t* z3 = nullptr;
  int64_t n3 = 0;
};
// One launch: cent = init (when the pointers differ), c_sq = row squared
// norms of init (the bits of launch_row_sqnorm), and the zero-fills.
int launch_lloyd_prologue(const void* init, void* cent, float* c_sq,
                          int64_t rows, int64_t D, int dtype,
                          const ZeroFill& f, hipStream_t s);
// p[b*N + n] = n for every batch row b.
int launch_iota_i32(int32_t* p, int64_t B, int64_t N, hipStream_t s);
int launch_fill_f32(float* p, float v, int64_t n, hipStream_t s);
int launch_fill_f64(double* p, double v, int64_t n, hipStream_t s);
int launch_converge_check(const float* shift, int it, float tol, int32_t* ctrl,
                          hipStream_t s);

// FKC_ASSIGN_FORCE_SAFE=1|true: route every dtype to the fp32 VALU kernel.
bool force_safe_assign();
// ---------------------------------------------------------------- quality
size_t quality_workspace_bytes(int64_t B, int64_t N, int64_t K);
// inertia (B doubles) and empty (one int: k empty in every row) are device
// pointers, either NULL.  sidx (optional, N entries shared by every row):
// the rows are samples x[:, sidx]; a row whose index is outside [0, sN)
// adds nothing.
int launch_quality(const void* x, const void* c, const int32_t* ids,
                   int64_t B, int64_t N, int64_t K, int64_t D, int dtype,
                   double* inertia, int32_t* empty, void* ws, size_t ws_bytes,
                   hipStream_t s, const int32_t* sidx = nullptr,
                   int64_t sN = 0);
// Nearest-centroid inertia of the S sampled points idx[0..S) of every row.
size_t sample_workspace_bytes(int64_t B, int64_t S, int64_t K, int64_t D,
                              int dtype);
int launch_sampled_inertia(const void* x, const void* c, const int32_t* idx,
                           int64_t S, int64_t B, int64_t N, int64_t K,
                           int64_t D, int dtype, double* inertia, void* ws,
                           size_t ws_bytes, hipStream_t s);

// ---------------------------------------------------------------- loop
// The Lloyd loop behind fkc_kmeans_lloyd*; profile = false ignores the
// profiling hook (creates no events).
int lloyd_run(const void* x, const void* init, void* centroids,
              int32_t* cluster_ids, int64_t B, int64_t N, int64_t K,
              int64_t D, int dtype, int max_iters, float tol, void* workspace,
              size_t workspace_bytes, fkc_stream_t stream,
              int32_t* n_iters_dev, int32_t* n_iters_host, bool profile);

// ---------------------------------------------------------------- device
// Compute units and the LDS one workgroup may hold on the current device,
// read with hipDeviceGetAttribute once per device.  The launch plans size
// their grids from it (workgroups that fill the chip, grids resident at
// once, centroid tables that fit LDS).  Without a device (a CPU host asking
// for workspace sizes) the MI355X figures stand in.  FKC_CUS=n overrides
// the CU count (tests and A/B runs of the plans of a smaller part).
constexpr int kMi355xCUs = 256;
constexpr int kMi355xLds = 160 * 1024;
struct DeviceShape {
  int cus;
  int lds_per_wg;
};
DeviceShape device_shape();

// FKC_NTILES=1|2|4|8: 16-point tiles per wave in the MFMA kernel; 0 = auto.
int ntiles_override();
// FKC_KSPLIT=1..64: centroid slices of a sliced MFMA assign; 0 = auto.
int ksplit_override();
// FKC_SAVE=0|1: saved-score fold of the four-tile D = 97..128 assign off /
// on where it exists; -1 = auto.
int save_override();
// FKC_RESIDENT=0|1: centroid-resident assign off / on where the table fits
// in LDS; -1 = auto.
int resident_override();
// FKC_UPDATE_ROWS=32|64|128: sorted rows per unit of the centroid update;
// 0 = auto.
int update_rows_override();
// FKC_UPDATE_SCAN=0|1: sort-free loop update off / on where it can run;
// -1 = auto.
int update_scan_override();
// FKC_SCAN_WGS=n (1..65536): size the sort-free update's grid to about n
// workgroups instead of one per CU; 0 = auto.
int scan_wgs_override();

}  // namespace fkc
