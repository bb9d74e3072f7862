/*
 * fkc.h — C ABI of the MI355X (gfx950) K-Means hot path.
 *
 * Batched Euclidean Lloyd iterations: assign -> stable label sort ->
 * indexed centroid update -> finalize.  Every entry point:
 *   - takes plain device pointers, element counts and a HIP stream
 *     (NULL = the null stream); nothing here knows about torch types;
 *   - enqueues asynchronously on that stream and never synchronises,
 *     except fkc_kmeans_lloyd when the caller asks for the host
 *     iteration count (see there);
 *   - allocates no device memory: scratch comes in through a caller-owned
 *     workspace whose size the matching *_workspace_bytes() reports and
 *     whose base is 256-byte aligned (hipMalloc pointers are);
 *   - returns FKC_OK (0) or a non-zero FKC_ERR_* code and never throws;
 *     fkc_last_error() then gives a message (thread-local).
 *
 * Layouts are the reference's: x (B,N,D) row-major, centroids (B,K,D),
 * ids (B,N) int32, sums (B,K,D) fp32, counts (B,K) int32, x_sq (B,N) fp32,
 * c_sq (B,K) fp32.  Element type is one of FKC_F32 / FKC_F16 / FKC_BF16.
 *
 * Reference interfaces replaced (OpsiClear/flash-kmeans-cuda):
 *   flash_kmeans_cuda/csrc/flash_kmeans_cuda.h:33-75  (fkc:: libtorch API)
 *   flash_kmeans_cuda/csrc/bindings.cpp:107-127        (_C extension module)
 *   flash_kmeans_cuda/kmeans.py:108-195                (Lloyd driver loop)
 *   flash_kmeans_cuda/ops.py:58-112                    (torch.sort call site)
 *   benchmarks/quality_compare.py:69-116               (quality evaluator)
 */
#ifndef FKC_H_
#define FKC_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(_WIN32)
#define FKC_CAPI __declspec(dllexport)
#else
#define FKC_CAPI __attribute__((visibility("default")))
#endif

/* Same type as hipStream_t (struct ihipStream_t*); NULL is the null stream. */
typedef struct ihipStream_t* fkc_stream_t;

enum fkc_status {
  FKC_OK = 0,
  FKC_ERR_INVALID = 1,     /* bad argument: shape, dtype, null pointer */
  FKC_ERR_WORKSPACE = 2,   /* workspace missing or smaller than required */
  FKC_ERR_LAUNCH = 3,      /* a HIP launch or runtime call failed */
  FKC_ERR_UNSUPPORTED = 4  /* valid request this build cannot serve */
};

enum fkc_dtype { FKC_F32 = 0, FKC_F16 = 1, FKC_BF16 = 2 };

/* Message for the last failing call on this thread ("" if none). */
FKC_CAPI const char* fkc_last_error(void);
/* Library version string, e.g. "0.1.0". */
FKC_CAPI const char* fkc_version(void);

/*
 * Nearest-centroid assignment: ids[b,n] = argmin_k ||x[b,n]-c[b,k]||^2,
 * the lowest k winning exact ties.
 * Replaces fkc::euclid_assign_out (flash_kmeans_cuda.h:41-46, api.cpp:58-72)
 * and _C.euclid_assign (bindings.cpp:43-63).
 *   - fp16/bf16 with D % 8 == 0 and D <= 512: MFMA kernel ranking
 *     c_sq[k] - 2<x,c_k> in fp32 (x_sq is not read; like the reference's
 *     raw-distance route, assign_sm80.cu:437-441, 687).
 *   - every other case, and FKC_ASSIGN_FORCE_SAFE=1: fp32 VALU kernel ranking
 *     max(0, x_sq + c_sq - 2<x,c>) (assign_safe.cu:55-80,
 *     assign_common.cuh:33-36).  x_sq may be NULL: then it is computed.
 * c_sq must hold the fp32 squared norms of the centroids as stored.
 */
FKC_CAPI int fkc_euclid_assign(const void* x, const void* centroids,
                               const float* x_sq, const float* c_sq,
                               int32_t* cluster_ids, int64_t B, int64_t N,
                               int64_t K, int64_t D, int dtype,
                               fkc_stream_t stream);

/*
 * Workspace variant of fkc_euclid_assign, same labels.  When the point
 * tiles of a shape cannot fill the GPU (fewer than ~1024 workgroups: N of
 * a few 100K or less with K > 512 at D = 128), the MFMA route cuts K into
 * slices scored by separate workgroups and merges their winners (first
 * maximum in slice order, so the lowest index still wins exact ties); the
 * workspace holds the partial winners, 8 bytes per point and slice.
 * fkc_euclid_assign_workspace_bytes returns the bytes needed (0: the shape
 * is not sliced and the workspace may be NULL); the workspace is 256-byte
 * aligned and may be reused once the call's stream work is done.  Same
 * reference interfaces as fkc_euclid_assign (flash_kmeans_cuda.h:41-46,
 * bindings.cpp:43-63); the slicing has no counterpart there (the reference
 * picks among tile shapes per dtype, D and K, assign_sm80.cu:707-1111).
 */
FKC_CAPI size_t fkc_euclid_assign_workspace_bytes(int64_t B, int64_t N,
                                                  int64_t K, int64_t D,
                                                  int dtype);
FKC_CAPI int fkc_euclid_assign_ws(const void* x, const void* centroids,
                                  const float* x_sq, const float* c_sq,
                                  int32_t* cluster_ids, int64_t B, int64_t N,
                                  int64_t K, int64_t D, int dtype,
                                  void* workspace, size_t workspace_bytes,
                                  fkc_stream_t stream);

/* out[r] = sum_d float(src[r,d])^2 for r < rows.  Replaces the torch
 * expressions (c.float()**2).sum(-1) at kmeans.py:94 and x.float()**2 at
 * kmeans.py:151. */
FKC_CAPI int fkc_row_sqnorm(const void* src, float* out, int64_t rows,
                            int64_t D, int dtype, fkc_stream_t stream);

/*
 * Stable sort of the labels of each batch row: sorted_ids[b,:] ascending,
 * perm[b,p] the original index of sorted position p, equal labels in index
 * order.  Labels outside [0,K) sort after every valid label, in index order.
 * Replaces torch.sort(cluster_ids, dim=1) at ops.py:89 (the reference asks
 * stable=False; this sort is always stable).
 * The output is always valid.  Each pass chains its key tiles with bounded
 * waits (decoupled look-back, and a row barrier where the first pass counts
 * the digits); a tile whose wait runs out recounts what it waited for from
 * the pass's input instead, which gives the same result.  The workspace's
 * first int32, cleared by every call, counts those recounts (0 in a normal
 * run; a diagnostic, not an error).
 */
FKC_CAPI size_t fkc_label_sort_workspace_bytes(int64_t B, int64_t N,
                                               int64_t K);
FKC_CAPI int fkc_label_sort(const int32_t* cluster_ids, int32_t* sorted_ids,
                            int32_t* perm, int64_t B, int64_t N, int64_t K,
                            void* workspace, size_t workspace_bytes,
                            fkc_stream_t stream);

/*
 * Centroid accumulation over label-sorted rows.  Adds into sums/counts
 * (the caller zeroes them first, as _C.centroid_update_sorted expects,
 * bindings.cpp:73-90); labels outside [0,K) are skipped
 * (update_sorted.cu:95,167).  Each maximal run of equal consecutive labels
 * adds its fp32 row sum (rows in sorted order) and its length with atomic
 * adds (update_sorted.cu:105,109), so any label order gives the right
 * totals.  When the rows of each valid label are contiguous (sorted labels,
 * invalid ones anywhere outside those runs) every bin gets exactly one add
 * and the result is deterministic: the same inputs give the same bits.
 * _sorted reads x_sorted row p for sorted position p (update_sorted.cu:39-116);
 * _indexed reads x row sorted_idx[p] (update_sorted.cu:118-186).
 */
FKC_CAPI size_t fkc_update_workspace_bytes(int64_t B, int64_t N, int64_t D);
FKC_CAPI int fkc_centroid_update_sorted(const void* x_sorted,
                                        const int32_t* ids_sorted, float* sums,
                                        int32_t* counts, int64_t B, int64_t N,
                                        int64_t K, int64_t D, int dtype,
                                        void* workspace, size_t workspace_bytes,
                                        fkc_stream_t stream);
FKC_CAPI int fkc_centroid_update_sorted_indexed(
    const void* x, const int32_t* sorted_idx, const int32_t* ids_sorted,
    float* sums, int32_t* counts, int64_t B, int64_t N, int64_t K, int64_t D,
    int dtype, void* workspace, size_t workspace_bytes, fkc_stream_t stream);

/*
 * out[b,k,:] = counts[b,k] > 0 ? cast(sums[b,k,:] / counts[b,k]) : old[b,k,:]
 * (IEEE division, round-to-nearest-even cast).  out may alias old.
 * Replaces fkc::centroid_finalize_out (flash_kmeans_cuda.h:71-75) and
 * launch_centroid_finalize (update_finalize.cu:39-121).
 */
FKC_CAPI int fkc_centroid_finalize(const float* sums, const int32_t* counts,
                                   const void* old_centroids, void* out,
                                   int64_t B, int64_t K, int64_t D, int dtype,
                                   fkc_stream_t stream);

/*
 * Clustering quality of labelled points, on the device (the evaluator of the
 * reference's benchmarks/quality_compare.py:69-90, `_assigned_inertia` and
 * `_empty_clusters`):
 *   inertia[b] = sum_n sum_d (float(x[b,n,d]) - float(c[b,ids[b,n],d]))^2,
 *                difference and square in fp32, sum in fp64 (the reference
 *                returns the sum over b);
 *   *empty_clusters = number of k in [0,K) that no point of any batch row
 *                carries (the reference counts the flattened labels into one
 *                K-bin histogram, `bincount(ids.reshape(-1)) == 0`).
 * Rows labelled outside [0,K) add nothing and are not counted.  inertia (B
 * doubles) and empty_clusters (one int32) are device pointers; either may be
 * NULL (x and centroids may then be NULL too when inertia is).  The result
 * is bitwise reproducible (fixed summation order).
 */
FKC_CAPI size_t fkc_quality_workspace_bytes(int64_t B, int64_t N, int64_t K);
FKC_CAPI int fkc_assigned_inertia(const void* x, const void* centroids,
                                  const int32_t* cluster_ids, int64_t B,
                                  int64_t N, int64_t K, int64_t D, int dtype,
                                  double* inertia, int32_t* empty_clusters,
                                  void* workspace, size_t workspace_bytes,
                                  fkc_stream_t stream);

/*
 * Inertia of a point sample (`_sample_exact_inertia`,
 * benchmarks/quality_compare.py:91-116): inertia[b] = sum over the S indices
 * n = sample_idx[s] (device int32, the same indices in every batch row) of
 * the squared distance from x[b,n] to its nearest centroid of row b.  The
 * nearest centroid is the assignment's (fkc_euclid_assign) and the distance
 * is summed as in fkc_assigned_inertia (fp32 differences and squares, fp64
 * total); the reference forms x_sq + c_sq - 2<x,c> in fp32 and takes its
 * minimum, clamped at 0, which agrees up to fp32 rounding.  An index outside
 * [0,N) adds nothing.  inertia: B device doubles.
 */
FKC_CAPI size_t fkc_sampled_inertia_workspace_bytes(int64_t B, int64_t S,
                                                    int64_t K, int64_t D,
                                                    int dtype);
FKC_CAPI int fkc_sampled_inertia(const void* x, const void* centroids,
                                 const int32_t* sample_idx, int64_t S,
                                 int64_t B, int64_t N, int64_t K, int64_t D,
                                 int dtype, double* inertia, void* workspace,
                                 size_t workspace_bytes, fkc_stream_t stream);

/*
 * Whole Lloyd loop of batch_kmeans_Euclid (kmeans.py:108-195) in one call.
 * centroids (B,K,D) holds the initial centroids on entry and the final ones
 * on return (updated in place); cluster_ids receives the labels of the last
 * assignment, made against the centroids before the last update
 * (kmeans.py:179-195).  With tol > 0 the loop stops after the first
 * iteration whose max centroid shift max_{b,k} ||new-old||_2 is below tol
 * (kmeans.py:104,190); the test runs on the device, so no host sync is
 * needed between iterations.  n_iters_dev (device int32, may be NULL)
 * receives the iterations run.  n_iters_host (may be NULL): when tol > 0 the
 * call synchronises the stream to fill it; when tol <= 0 it is max_iters.
 */
FKC_CAPI size_t fkc_kmeans_workspace_bytes(int64_t B, int64_t N, int64_t K,
                                           int64_t D, int dtype,
                                           int max_iters);
FKC_CAPI int fkc_kmeans_lloyd(const void* x, void* centroids,
                              int32_t* cluster_ids, int64_t B, int64_t N,
                              int64_t K, int64_t D, int dtype, int max_iters,
                              float tol, void* workspace,
                              size_t workspace_bytes, fkc_stream_t stream,
                              int32_t* n_iters_dev, int32_t* n_iters_host);
/*
 * fkc_kmeans_lloyd with the initial centroids read from init_centroids (left
 * unmodified; it is either the same buffer as centroids or does not overlap
 * it) and the final ones written to centroids.  The copy is part of the loop's first launch, so a
 * caller that keeps its initial centroids intact needs no separate copy
 * (the reference's loop ping-pongs into init_centroids' storage,
 * kmeans.py:157-193; this package's batch_kmeans_Euclid never writes it).
 * Same workspace as fkc_kmeans_lloyd.
 */
FKC_CAPI int fkc_kmeans_lloyd_from(const void* x, const void* init_centroids,
                                   void* centroids, int32_t* cluster_ids,
                                   int64_t B, int64_t N, int64_t K, int64_t D,
                                   int dtype, int max_iters, float tol,
                                   void* workspace, size_t workspace_bytes,
                                   fkc_stream_t stream, int32_t* n_iters_dev,
                                   int32_t* n_iters_host);

/*
 * fkc_kmeans_lloyd_from without a workspace argument and without any device
 * allocation: no counterpart in the reference; it is for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  The loop's workspace is a static device array of
 * fkc_kmeans_noalloc_max_bytes() bytes (64 MiB) that each GPU using the
 * library holds until the process ends; a shape whose workspace
 * (fkc_kmeans_workspace_bytes) is larger is refused with FKC_ERR_WORKSPACE.
 * The array is looked up once per device, on the first call made with that
 * device current; stream must belong to the current device.  Every call on
 * one GPU shares the array: calls that overlap on one GPU (other streams or
 * host threads) race, so serialise them.  Same results as
 * fkc_kmeans_lloyd_from; the profiling hook is not applied.  Under HIP graph
 * capture: make the device's first call outside the capture (it looks the
 * array up), pass tol <= 0 and n_iters_host = NULL (with tol > 0 filling
 * n_iters_host synchronises the stream, which capture forbids); n_iters_dev
 * may be given.
 */
FKC_CAPI size_t fkc_kmeans_noalloc_max_bytes(void);
FKC_CAPI int fkc_kmeans_lloyd_noalloc(const void* x, const void* init_centroids,
                                      void* centroids, int32_t* cluster_ids,
                                      int64_t B, int64_t N, int64_t K,
                                      int64_t D, int dtype, int max_iters,
                                      float tol, fkc_stream_t stream,
                                      int32_t* n_iters_dev,
                                      int32_t* n_iters_host);

/*
 * Profiling hook for benchmarks (no counterpart in the reference): with
 * enable = k > 0, fkc_kmeans_lloyd times the assignment launch of the middle
 * iteration of every run of k loop iterations (iterations k/2, k/2 + k,
 * k/2 + 2k, ..., integer division) with HIP events stamped by the launch's
 * dispatch on its stream (each timed launch costs the stream a few
 * microseconds, so k > 1 keeps that out of most iterations); enable = 0
 * turns it off.  fkc_profile_assign_ms() synchronises on the recorded events
 * and returns the summed assignment time in ms and the timed launch count.
 * The hook is process-wide: calls from several threads are safe and their
 * timed launches are pooled.
 */
FKC_CAPI void fkc_profile_enable(int enable);
FKC_CAPI int fkc_profile_assign_ms(double* total_ms, int64_t* launches);

/*
 * Diagnostic (no counterpart in the reference): byte offset, inside a
 * workspace of fkc_kmeans_workspace_bytes(B, N, K, D, dtype, max_iters)
 * bytes, of an int32 that fkc_kmeans_lloyd* clear at the start of a call and
 * that counts the label-sort tiles of that call whose bounded wait on other
 * tiles ran out, so that they recounted from their input instead (the
 * results are the same either way; a non-zero count means the sort's grid
 * did not run at once, e.g. on a GPU shared with other work, and cost
 * time).  Read it after the call has finished (one int32 copy to the host).
 */
FKC_CAPI size_t fkc_kmeans_sort_recounts_offset(int64_t B, int64_t N, int64_t K,
                                                int64_t D, int dtype,
                                                int max_iters);

#ifdef __cplusplus
}
#endif

#endif /* FKC_H_ */
