// Centroid sums and counts over label-sorted rows, deterministic.
//
// Restates the run semantics of the reference accumulator
// (flash_kmeans_cuda/csrc/update/update_sorted.cu:39-186): rows sorted by
// label form runs of equal labels; each run contributes its fp32 column sums
// and its length to sums[b,label,:] and counts[b,label]; labels outside
// [0,K) are skipped (:95, :167).  The reference flushes every run with fp32
// atomicAdd, so its sums depend on scheduling.  Here every bin has exactly
// one writer and rows are summed in sorted order, so results are bitwise
// reproducible:
//
//   update_runs  : one wave per unit of 128 consecutive sorted rows (64 or
//                  32 when N is small, for parallelism).  Lanes
//                  own column slices (64 lanes x VEC x NI columns per pass
//                  over the row), so every row is one coalesced load per
//                  lane slice; a unit's labels and permutation entries are
//                  loaded up front, then rows are fetched 32 / NI at a time
//                  (through the permutation for the indexed variant) before
//                  being folded into the run accumulator.  A run wholly inside the unit is
//                  written directly.  A run entering from the previous unit
//                  ("head") or leaving into the next ("tail") is parked in a
//                  per-unit partial slot instead.
//   update_blocks: a run can span many units (few clusters, many points).
//                  For every block of 64 units that lies wholly inside one
//                  run, one wave adds the block's 64 head partials in unit
//                  order into a block partial.  In the Lloyd loop this is
//                  done inside update_runs instead: the last of a block's
//                  64 through-units to finish (an arrival counter) sums the
//                  block, with the same order and bits.
//   update_merge : the unit where a multi-unit run starts owns it.  It finds
//                  the run's last unit by ballots over unit and block flags,
//                  then adds, in unit order, its tail partial, the heads of
//                  the following units in its own block, the partials of the
//                  blocks the run covers, and the heads of the units of the
//                  block where the run ends; the bin is written once.  A run
//                  over L units adds at most 127 + L/64 partial rows, 32 rows
//                  in flight per wave (four lane groups, eight rows each).
//
// Mode "add" (the _C / C-ABI contract) adds into caller-zeroed outputs with
// atomic adds, so it is correct for labels in any order, as the reference's
// atomics are: a label whose rows are not contiguous (unsorted input, or
// invalid labels between its rows) forms several runs that each add their
// share.  With sorted input every bin still gets exactly one add, so the
// result is the same bits on every run.  Mode "overwrite" (the Lloyd loop,
// where every label is valid and sorted) stores, and the run start of each
// label also zeroes the empty bins below it, so no separate clearing pass is
// needed.
#include "device_util.hpp"
#include "fkc_internal.hpp"

#include <limits.h>

#include <type_traits>

namespace fkc {
namespace {

constexpr int UR_MAX = 128;  // sorted rows per unit (one wave), at most

// Rows per unit: 128 when that still gives >= 2048 units (512 workgroups),
// else 64, else 32 — small N needs the extra waves to hide its latency.
// FKC_UPDATE_ROWS=32|64|128 overrides (A/B runs; the workspace query and
// the launch read it alike).
int choose_ur(int64_t B, int64_t N) {
  if (const int o = update_rows_override()) return o;
  for (int ur = UR_MAX; ur > 32; ur >>= 1)
    if (B * ((N + ur - 1) / ur) >= 2048) return ur;
  return 32;
}
constexpr int UT = 256;  // threads per workgroup: 4 units
constexpr int UB = 64;   // units per block of the two-level run merge

// VEC consecutive columns of one row as one raw load (VEC in {1, 2}), and
// their conversion to fp32.
template <int DT, int VEC>
struct RawCols;
template <int VEC>
struct RawCols<FKC_F32, VEC> {
  using T = typename std::conditional<VEC == 2, float2, float>::type;
  __device__ static T load(const float* p) { return *reinterpret_cast<const T*>(p); }
  __device__ static T zero() { return T{}; }
  // Store VEC elements as one access.
  __device__ static void store(float* p, const float* e) {
    if constexpr (VEC == 2)
      *reinterpret_cast<float2*>(p) = float2{e[0], e[1]};
    else
      *p = e[0];
  }
  __device__ static void cvt(T r, float* out) {
    if constexpr (VEC == 2) {
      out[0] = r.x;
      out[1] = r.y;
    } else {
      out[0] = r;
    }
  }
};
template <int DT, int VEC>
struct RawCols {  // 16-bit element types
  using E = Elem<DT>;
  using T = typename std::conditional<VEC == 2, uint32_t, uint16_t>::type;
  __device__ static T load(const typename E::T* p) {
    return *reinterpret_cast<const T*>(p);
  }
  __device__ static T zero() { return 0; }
  // Store VEC elements as one access.
  __device__ static void store(typename E::T* p, const typename E::T* e) {
    uint32_t bits = 0;
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      uint16_t h;
      __builtin_memcpy(&h, &e[v], 2);
      bits |= (uint32_t)h << (16 * v);
    }
    *reinterpret_cast<T*>(p) = (T)bits;
  }
  __device__ static void cvt(T r, float* out) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      const uint16_t h = (uint16_t)((uint32_t)r >> (16 * v));
      typename E::T e;
      __builtin_memcpy(&e, &h, 2);
      out[v] = E::load(e);
    }
  }
};

struct UnitMeta {  // per unit, int32 x 4
  enum { TAIL_ID = 0, TAIL_LEN = 1, HEAD_LEN = 2, THROUGH = 3 };
};

// Block partials computed inside update_runs (null ctr: update_blocks
// computes them).  Flags of full blocks are set to tag.
struct BlockArgs {
  float* part;    // [B][nblocks][D]
  int32_t* meta;  // [B][nblocks][2]: flag, row count
  int32_t* ctr;   // [B][nblocks][column blocks] arrival counters
  int nblocks;
  int tag;
};

constexpr int FIN_DMAX = 512;  // widest row the fused finalize handles

// Finalize fused into the update (the Lloyd loop): where a bin's final sum
// is known, the wave that holds it computes the new centroid row at once,
// exactly as finalize_kernel (finalize.hip) would from the stored sums:
// new = cast(sum / count) with IEEE division, c_sq = sum of new^2 and the
// row's shift ||new - old||_2, accumulated in the column order shared with
// finalize_kernel and row_sqnorm (lane l: columns VEC*(l + 64 i) + v, fma in
// (i, v) order) and added over lanes by row_sum, so every bit matches the
// separate kernels.  Empty bins are left alone: their centroid, c_sq and
// zero shift stand.
template <typename T>
struct FinArgs {
  T* cent;          // (B, K, D) centroids, updated in place; null: not fused
  float* c_sq;      // (B, K) next iteration's c_sq
  float* shift;     // this iteration's max shift (float bits), may be null
};

// The lanes of one wave wrote `row` in LDS; make the writes visible to the
// wave's own later reads of other lanes' entries (compiler ordering, and
// LDS counter drained; global loads in flight are not waited for).
__device__ inline void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0) only
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// c_sq and (when wanted) the shift of a finalized row from the lanes'
// partial sums.
__device__ inline void finish_norms(float sq, float sh, float* csq,
                                    float* shift, int lane) {
  sq = row_sum(sq);
  if (lane == 0) *csq = sq;
  if (shift != nullptr) {
    sh = row_sum(sh);
    if (lane == 0)
      atomicMax(reinterpret_cast<unsigned int*>(shift), __float_as_uint(sqrtf(sh)));
  }
}

// Finalize from a row of sums in LDS (the run merge).  The old row is read
// only when the shift is wanted.
template <int DT>
__device__ inline void finalize_row(const float* row, int cnt,
                                    typename Elem<DT>::T* crow, float* csq,
                                    float* shift, int D, int lane) {
  using E = Elem<DT>;
  const float fc = (float)cnt;
  const int vec = row_vec(D);
  float sq = 0.f, sh = 0.f;
  for (int c = vec * lane; c < D; c += vec * 64) {
    for (int v = 0; v < vec; ++v) {
      const int d = c + v;
      const typename E::T n = E::store(row[d] / fc);
      const float nf = E::load(n);
      if (shift != nullptr) {
        const float df = nf - E::load(crow[d]);
        sh = fmaf(df, df, sh);
      }
      crow[d] = n;
      sq = fmaf(nf, nf, sq);
    }
  }
  finish_norms(sq, sh, csq, shift, lane);
}

// A run's unit partials merged and the row finalized in one pass, lane by
// lane over finalize_row's columns.  part holds the tail (slot 0) and the n
// heads in item order (slots 1..n), in LDS; each column is summed with
// wave_ordered_sum's bracketing (four groups, group g adding items g, g+4,
// ... in order to a zero start, the tail starting group 0, then the groups
// added in order), so the row gets the bits of wave_ordered_sum followed by
// finalize_row, without the row buffer or the lane exchanges.
template <int DT>
__device__ inline void merge_finalize(const float* part, int n, int cnt,
                                      typename Elem<DT>::T* crow, float* csq,
                                      float* shift, int D, int lane) {
  using E = Elem<DT>;
  const float fc = (float)cnt;
  const int vec = row_vec(D);
  float sq = 0.f, sh = 0.f;
  for (int c = vec * lane; c < D; c += vec * 64) {
    for (int v = 0; v < vec; ++v) {
      const int d = c + v;
      const float* it = part + D + d;
      float g0 = part[d], g1 = 0.f, g2 = 0.f, g3 = 0.f;
      int i = 0;
      for (; i + 4 <= n; i += 4) {
        g0 += it[i * D];
        g1 += it[(i + 1) * D];
        g2 += it[(i + 2) * D];
        g3 += it[(i + 3) * D];
      }
      if (i < n) g0 += it[i * D];
      if (i + 1 < n) g1 += it[(i + 1) * D];
      if (i + 2 < n) g2 += it[(i + 2) * D];
      const float tot = ((g0 + g1) + g2) + g3;
      const typename E::T nv = E::store(tot / fc);
      const float nf = E::load(nv);
      if (shift != nullptr) {
        const float df = nf - E::load(crow[d]);
        sh = fmaf(df, df, sh);
      }
      crow[d] = nv;
      sq = fmaf(nf, nf, sq);
    }
  }
  finish_norms(sq, sh, csq, shift, lane);
}

// Wave-cooperative ordered sum of partial rows (D fp32 each):
//   out[c] = first[c] + row(0)[c] + ... + row(n-1)[c]   (first may be null)
// for the columns c in [c_lo, c_hi).  The wave splits into G lane groups;
// group g sums rows i = g, g+G, g+2G ... in increasing i (eight loads in
// flight per lane before their adds) over V-wide column vectors, then the
// group sums are added in group order.  The bracketing depends only on n,
// so the result is reproducible bit for bit (and a column's bits do not
// depend on the range it is summed in).  Mode 0 stores out, mode 1 adds
// into it atomically.  COHERENT reads the rows with agent-scope atomic
// loads: rows another workgroup of the same launch stored with agent-scope
// atomic stores.
template <int V, bool COHERENT>
__device__ inline void ld_cols(const float* p, float* o) {
  if constexpr (COHERENT) {
#pragma unroll
    for (int v = 0; v < V; ++v)
      o[v] = __hip_atomic_load(p + v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else if constexpr (V == 4) {
    const float4 v = *reinterpret_cast<const float4*>(p);
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
  } else {
    o[0] = p[0];
  }
}

template <int V, bool COHERENT = false, typename RowFn>
__device__ inline void wave_ordered_sum(const float* first, int n, int c_lo,
                                        int c_hi, RowFn row, float* out,
                                        int add, int lane) {
  constexpr int G = 4, LG = 64 / G, PF = 8;
  const int g = lane / LG, sub = lane % LG;
  for (int c0 = c_lo; c0 < c_hi; c0 += LG * V) {
    const int c = c0 + sub * V;
    const bool cok = c < c_hi;  // (c_hi - c_lo) % V == 0: whole vectors
    float acc[V];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = 0.f;
    if (first != nullptr && g == 0 && cok) ld_cols<V, false>(first + c, acc);
    for (int i0 = g; i0 < n; i0 += G * PF) {
      float t[PF][V];
#pragma unroll
      for (int j = 0; j < PF; ++j) {
        const int i = i0 + j * G;
        if (cok && i < n) {
          ld_cols<V, COHERENT>(row(i) + c, t[j]);
        } else {
#pragma unroll
          for (int v = 0; v < V; ++v) t[j][v] = 0.f;
        }
      }
#pragma unroll
      for (int j = 0; j < PF; ++j)
        if (i0 + j * G < n) {
#pragma unroll
          for (int v = 0; v < V; ++v) acc[v] += t[j][v];
        }
    }
    float tot[V];
#pragma unroll
    for (int v = 0; v < V; ++v) tot[v] = __shfl(acc[v], sub, 64);
#pragma unroll
    for (int gg = 1; gg < G; ++gg)
#pragma unroll
      for (int v = 0; v < V; ++v) tot[v] += __shfl(acc[v], gg * LG + sub, 64);
    if (g == 0 && cok) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        if (add)
          unsafeAtomicAdd(out + c + v, tot[v]);
        else
          out[c + v] = tot[v];
      }
    }
  }
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Wpass-failed"
template <int DT, int VEC, int NI, bool INDEXED>
__global__ void __launch_bounds__(UT)
update_runs_kernel(const typename Elem<DT>::T* __restrict__ x,
                   const int32_t* __restrict__ perm,
                   const int32_t* __restrict__ sids, float* __restrict__ sums,
                   int32_t* __restrict__ counts, float* __restrict__ part,
                   int32_t* __restrict__ meta, int N, int K, int D,
                   int nunits, int ur, int overwrite, BlockArgs blk,
                   FinArgs<typename Elem<DT>::T> fin,
                   const int32_t* __restrict__ ctrl) {
  using T = typename Elem<DT>::T;
  using E = Elem<DT>;
  using RC = RawCols<DT, VEC>;
  if (loop_done(ctrl)) return;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform
  const int b = blockIdx.y;
  const int u = blockIdx.x * (UT / 64) + wave;
  if (u >= nunits) return;
  const bool lead = blockIdx.z == 0;  // column block 0 writes counts / meta
  const int cbase = blockIdx.z * (64 * VEC * NI);
  const int p0 = u * ur;
  const int p1 = min(p0 + ur, N);

  const bool fused = fin.cent != nullptr;  // uniform
  // With the shift wanted, the old centroid row of each run's label is
  // loaded when the run starts (the label's row is finalized, if here, only
  // by this wave: a label is one contiguous run).
  const bool pref = fused && fin.shift != nullptr;  // uniform
  const int32_t* ib = sids + (size_t)b * N;
  const int32_t* pb = INDEXED ? perm + (size_t)b * N : nullptr;
  const T* xb = x + (size_t)b * N * D;
  float* sb = sums + (size_t)b * K * D;
  int32_t* cntb = counts + (size_t)b * K;
  float* partb = part + (size_t)b * nunits * 2 * D;

  const bool has_prev = p0 > 0, has_next = p1 < N;
  const int prev = has_prev ? ib[p0 - 1] : 0;
  const int next = has_next ? ib[p1] : 0;
  // Block partials in this launch: labels are sorted, so the unit's block
  // of UB units lies wholly inside one run exactly when the label before
  // its first row equals the label after its last row.
  bool bfull = false;  // wave-uniform
  if (blk.ctr != nullptr) {
    const int64_t bs = (int64_t)(u / UB) * UB * ur, be = bs + (int64_t)UB * ur;
    bfull = bs > 0 && be < N && ib[bs - 1] == ib[be];
  }

  int col[NI];
  bool cok[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    col[i] = cbase + (lane + 64 * i) * VEC;
    cok[i] = col[i] < D;  // D % VEC == 0, so the whole vector is in range
  }
  int lcol[NI];  // the column each lane loads: its own, or 0 past D
#pragma unroll
  for (int i = 0; i < NI; ++i) lcol[i] = cok[i] ? col[i] : 0;

  using Acc = float[NI][VEC];
  int tail_id = 0, tail_len = 0, head_len = 0, through = 0;

  // Zero sums/counts of bins [lo, hi) (overwrite mode only).
  auto zero_bins = [&](int lo, int hi) {
    lo = max(lo, 0);
    hi = min(hi, K);
    for (int k = lo; k < hi; ++k) {
#pragma unroll
      for (int i = 0; i < NI; ++i)
        if (cok[i]) {
#pragma unroll
          for (int v = 0; v < VEC; ++v) sb[(size_t)k * D + col[i] + v] = 0.f;
        }
    }
    if (lead)
      for (int k = lo + lane; k < hi; k += 64) cntb[k] = 0;
  };

  // coherent: agent-scope atomic stores, which another workgroup of this
  // launch may read (the block sum below).
  auto store_part = [&](int slot, const Acc& a, bool coherent) {
    float* dst = partb + ((size_t)u * 2 + slot) * D;
#pragma unroll
    for (int i = 0; i < NI; ++i)
      if (cok[i]) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          if (coherent)
            __hip_atomic_store(dst + col[i] + v, a[i][v], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
          else
            dst[col[i] + v] = a[i][v];
        }
      }
  };

  // Close the run of label `id` covering sorted rows [s, e) with sums `a`.
  auto flush = [&](int id, int s, int e, const Acc& a) {
    const bool continuing = s == p0 && has_prev && prev == id;
    const bool continued = e == p1 && has_next && next == id;
    if (continuing) {
      store_part(0, a, bfull);
      head_len = e - s;
      through = continued ? 1 : 0;
    } else if (continued) {
      store_part(1, a, false);
      tail_id = id;
      tail_len = e - s;
    } else if (fused && (uint32_t)id < (uint32_t)K) {
      // The run's sums are in the shared column order (the fused path has
      // one column block, so col[i] = VEC*(lane + 64 i)): finalize straight
      // from them.  The old row is read only when the shift is wanted.
      const float fc = (float)(e - s);
      T* crow = fin.cent + ((size_t)b * K + id) * D;
      float sq = 0.f, sh = 0.f;
#pragma unroll
      for (int i = 0; i < NI; ++i)
        if (cok[i]) {
          float of[VEC];
          if (pref) RC::cvt(RC::load(crow + col[i]), of);
          T nv[VEC];
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            nv[v] = E::store(a[i][v] / fc);
            const float nf = E::load(nv[v]);
            sq = fmaf(nf, nf, sq);
            if (pref) {
              const float df = nf - of[v];
              sh = fmaf(df, df, sh);
            }
          }
          RC::store(crow + col[i], nv);
        }
      finish_norms(sq, sh, fin.c_sq + (size_t)b * K + id,
                   pref ? fin.shift : nullptr, lane);
    } else if ((uint32_t)id < (uint32_t)K) {
      float* dst = sb + (size_t)id * D;
#pragma unroll
      for (int i = 0; i < NI; ++i)
        if (cok[i]) {
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            if (overwrite)
              dst[col[i] + v] = a[i][v];
            else
              unsafeAtomicAdd(dst + col[i] + v, a[i][v]);
          }
        }
      if (lead && lane == 0) {
        if (overwrite)
          cntb[id] = e - s;
        else
          atomicAdd(cntb + id, e - s);
      }
    }
  };

  // Labels and permutation entries of the unit's rows, one per lane per
  // 64-row chunk, loaded up front, and per chunk the mask of rows that start
  // a new run (never the unit's first row: its run is open from the start).
  constexpr int CH = UR_MAX / 64;
  int ivs[CH], pvs[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int p = p0 + c * 64 + lane;
    ivs[c] = p < p1 ? ib[p] : 0;
    pvs[c] = INDEXED ? (p < p1 ? pb[p] : 0) : p;
  }
  uint64_t starts[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    int before = __shfl_up(ivs[c], 1, 64);
    if (lane == 0)
      before = c == 0 ? ivs[0] : __builtin_amdgcn_readlane(ivs[c - 1], 63);
    const int p = p0 + c * 64 + lane;
    starts[c] = __builtin_amdgcn_ballot_w64(p < p1 && ivs[c] != before);
  }

  // Per chunk, each lane's row of the gather: its byte offset in the batch
  // row (row 0's where the row is past the unit or its permutation entry is
  // outside [0,N): read but not folded) and the ballot of rows folded.
  uint64_t goff[CH];
  uint64_t gok[CH];
  const char* xl[NI];  // this lane's column of row 0
#pragma unroll
  for (int i = 0; i < NI; ++i) xl[i] = reinterpret_cast<const char*>(xb + lcol[i]);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int p = p0 + c * 64 + lane;
    const bool ok = p < p1 && (uint32_t)pvs[c] < (uint32_t)N;
    goff[c] = (uint64_t)(uint32_t)(ok ? pvs[c] : 0) * (uint64_t)D * sizeof(T);
    gok[c] = __builtin_amdgcn_ballot_w64(ok);
  }

  int cur = __builtin_amdgcn_readfirstlane(ivs[0]);
  int rs = p0;
  if (overwrite && !fused && !(has_prev && prev == cur))
    zero_bins(has_prev ? prev + 1 : 0, cur);

  // Rows are gathered RB at a time (raw words in flight, converted when
  // folded) and folded in sub-batches of FH rows.  The fold is straight-line
  // code with no branch: at every row the running sums go to an LDS slot
  // (the next free slot when the row starts a run, else a scratch slot) and
  // restart from zero if the row starts a run.  The runs that closed in the
  // sub-batch are then flushed from their slots by a loop with a single
  // flush site.  (A per-row branch to a flush, even one that is rarely
  // taken, doubled the kernel's time; sub-batches without a run start take
  // a plain-add path instead.)
  constexpr int RB = 32 / NI;          // rows in flight per wave
  constexpr int FH = 16 / NI;          // rows per folded sub-batch
  constexpr int SL = NI * VEC;         // floats per lane per slot
  __shared__ float slot[UT / 64][FH + 1][SL][64];
  float (*wslot)[SL][64] = slot[wave];
  const int urows = p1 - p0;
  Acc acc;
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[i][v] = 0.f;

  using R = typename RC::T;
  // The full unroll asked here exceeds the unroller's size limit and is not
  // done (clang warns; the warning is silenced around this kernel), yet the
  // code built with the request ran 9% faster at N = 524288, D = 128 than
  // with `unroll 1` or `unroll 2` (34.8 vs 37.9 / 37.3 us).
#pragma unroll
  for (int q = 0; q < UR_MAX / RB; ++q) {
    const int r0 = q * RB;  // first unit row of the batch
    if (r0 >= urows) break;
    R raw[RB][NI];
    // Rows with a permutation entry in [0,N) inside the unit (bit jj: row
    // r0 + jj), from the chunk's ballot.
    const uint32_t okm =
        (uint32_t)(gok[r0 >> 6] >> (r0 & 63)) & (RB == 32 ? ~0u : (1u << RB) - 1u);
#pragma unroll
    for (int jj = 0; jj < RB; ++jj) {
      const int r = r0 + jj;  // a constant once unrolled
      // The row's byte offset, held by lane r % 64 of its chunk: two lane
      // reads, no per-row scalar arithmetic.
      const uint64_t lo = (uint32_t)__builtin_amdgcn_readlane(
          (int)(uint32_t)goff[r >> 6], r & 63);
      const uint64_t hi = (uint32_t)__builtin_amdgcn_readlane(
          (int)(uint32_t)(goff[r >> 6] >> 32), r & 63);
      const uint64_t off = (hi << 32) | lo;
      // Unconditional, from an in-bounds column: a lane past D loads column
      // 0 and its sums are never stored (every store checks cok), so no
      // per-row branch on the lane's column is needed.
#pragma unroll
      for (int i = 0; i < NI; ++i)
        raw[jj][i] = RC::load(reinterpret_cast<const T*>(xl[i] + off));
    }
#pragma unroll
    for (int h = 0; h < RB / FH; ++h) {
      const int s0 = r0 + h * FH;  // first unit row of the sub-batch
      if (s0 >= urows) break;
      const uint64_t cm = starts[s0 >> 6] >> (s0 & 63);
      const uint32_t hb = (uint32_t)cm & ((1u << FH) - 1u);  // run starts
      // A sub-batch with no run start and every row in use (most of them:
      // runs are long) only adds its rows, the same additions as below
      // without the slot stores and selects.  The branch is wave-uniform and
      // taken per sub-batch, not per row (measured at N = 524288, D = 128:
      // 34.4 -> 31.5 us; at c4's 8 x 65536 x 64: 32.8 -> 30.2 us).
      const uint32_t um = (okm >> (h * FH)) & ((1u << FH) - 1u);
      if (hb == 0u && um == (1u << FH) - 1u) {
#pragma unroll
        for (int t = 0; t < FH; ++t) {
          const int jj = h * FH + t;
#pragma unroll
          for (int i = 0; i < NI; ++i) {
            float f[VEC];
            RC::cvt(raw[jj][i], f);
#pragma unroll
            for (int v = 0; v < VEC; ++v) acc[i][v] = acc[i][v] + f[v];
          }
        }
        continue;
      }
      int nseg = 0;
#pragma unroll
      for (int t = 0; t < FH; ++t) {
        const int jj = h * FH + t;
        const bool st = (hb >> t) & 1u;  // wave-uniform
        const int sl = st ? nseg : FH;
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
          for (int v = 0; v < VEC; ++v) wslot[sl][i * VEC + v][lane] = acc[i][v];
        nseg += st ? 1 : 0;
        const bool use = (okm >> jj) & 1u;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          float f[VEC];
          RC::cvt(raw[jj][i], f);
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            const float base = st ? 0.f : acc[i][v];
            acc[i][v] = use ? base + f[v] : base;
          }
        }
      }
      if (hb != 0u) {
        wave_lds_sync();
        uint32_t m = hb;
#pragma unroll 1
        for (int k = 0; m != 0u; ++k) {
          const int t = __builtin_ctz(m);
          m &= m - 1u;
          const int r = s0 + t;  // unit row where the next run starts
          Acc a;
#pragma unroll
          for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int v = 0; v < VEC; ++v) a[i][v] = wslot[k][i * VEC + v][lane];
          flush(cur, rs, p0 + r, a);
          const int id = __builtin_amdgcn_readlane(r < 64 ? ivs[0] : ivs[CH - 1], r & 63);
          if (overwrite && !fused) zero_bins(cur + 1, id);
          cur = id;
          rs = p0 + r;
        }
      }
    }
  }
  flush(cur, rs, p1, acc);
  if (overwrite && !fused && !has_next) zero_bins(cur + 1, K);

  if (lead && lane == 0) {
    int32_t* m = meta + ((size_t)b * nunits + u) * 4;
    m[UnitMeta::TAIL_ID] = tail_id;
    m[UnitMeta::TAIL_LEN] = tail_len;
    m[UnitMeta::HEAD_LEN] = head_len;
    m[UnitMeta::THROUGH] = through;
  }

  // Block partials in this launch (the Lloyd loop): every unit of a block
  // that lies wholly inside one run arrives at the block's counter (one per
  // column block) once its head partial is stored; the UB-th arrival sums
  // the block's head partials, in the order and bracketing of
  // update_blocks_kernel, into the block partial.  Other blocks are not
  // touched; their flags keep an earlier tag.
  if (bfull) {
    // The head partial's atomic stores are performed where the summing
    // wave reads them; waiting for them orders them before the arrival.
    drain_before_announce();
    const int beta = u / UB;
    int old = 0;
    if (lane == 0)
      old = atomicAdd(blk.ctr + ((size_t)b * blk.nblocks + beta) * gridDim.z +
                          blockIdx.z,
                      1);
    old = __builtin_amdgcn_readfirstlane(old);
    if (old == UB - 1) {
      const int c_hi = min(cbase + 64 * VEC * NI, D);
      float* dst = blk.part + ((size_t)b * blk.nblocks + beta) * D;
      auto row = [&](int i) {
        return partb + ((size_t)(beta * UB + i) * 2 + 0) * D;
      };
      if (D % 4 == 0)
        wave_ordered_sum<4, true>(nullptr, UB, cbase, c_hi, row, dst, 0, lane);
      else
        wave_ordered_sum<1, true>(nullptr, UB, cbase, c_hi, row, dst, 0, lane);
      if (lead && lane == 0) {
        int32_t* bm = blk.meta + ((size_t)b * blk.nblocks + beta) * 2;
        bm[0] = blk.tag;
        bm[1] = UB * ur;
      }
    }
  }
}
#pragma clang diagnostic pop

// One wave per block of UB units.  A block whose every unit lies inside a
// single run ("full") gets the ordered sum of its head partials and its row
// count, and its flag word is set to `tag`; other blocks get flag 0.
__global__ void __launch_bounds__(UT)
update_blocks_kernel(const float* __restrict__ part,
                     const int32_t* __restrict__ meta,
                     float* __restrict__ bpart, int32_t* __restrict__ bmeta,
                     int D, int nunits, int nblocks, int tag,
                     const int32_t* __restrict__ ctrl) {
  if (loop_done(ctrl)) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.y;
  const int beta = blockIdx.x * (UT / 64) + wave;
  if (beta >= nblocks) return;
  const int32_t* mb = meta + (size_t)b * nunits * 4;
  const int v = beta * UB + lane;
  const bool thr = v < nunits && mb[(size_t)v * 4 + UnitMeta::THROUGH] != 0;
  const int hl = v < nunits ? mb[(size_t)v * 4 + UnitMeta::HEAD_LEN] : 0;
  const bool full = __builtin_amdgcn_ballot_w64(thr) == ~0ull;
  int32_t* bm = bmeta + ((size_t)b * nblocks + beta) * 2;
  const int len = wave_sum_i(hl);
  if (!full) {
    if (lane == 0) {
      bm[0] = 0;
      bm[1] = 0;
    }
    return;
  }
  const float* pb = part + (size_t)b * nunits * 2 * D;
  float* dst = bpart + ((size_t)b * nblocks + beta) * D;
  const int v0 = beta * UB;
  auto row = [&](int i) { return pb + ((size_t)(v0 + i) * 2 + 0) * D; };
  if (D % 4 == 0)
    wave_ordered_sum<4>(nullptr, UB, 0, D, row, dst, 0, lane);
  else
    wave_ordered_sum<1>(nullptr, UB, 0, D, row, dst, 0, lane);
  if (lane == 0) {
    bm[0] = tag;
    bm[1] = len;
  }
}

// One wave per unit; only units holding a tail partial (run owners) work.
template <int DT>
__global__ void __launch_bounds__(UT)
update_merge_kernel(const float* __restrict__ part,
                    const int32_t* __restrict__ meta,
                    const float* __restrict__ bpart,
                    const int32_t* __restrict__ bmeta, float* __restrict__ sums,
                    int32_t* __restrict__ counts, int K, int D, int nunits,
                    int nblocks, int overwrite, int tag,
                    int32_t* __restrict__ bctr, int nz,
                    FinArgs<typename Elem<DT>::T> fin,
                    const int32_t* __restrict__ ctrl) {
  __shared__ float fin_row[UT / 64][FIN_DMAX];
  if (loop_done(ctrl)) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.y;
  const int u = blockIdx.x * (UT / 64) + wave;
  if (u >= nunits) return;
  // The first unit of each block clears the block's arrival counters for
  // the next launch of update_runs (nothing in this launch reads them).
  if (bctr != nullptr && u % UB == 0)
    for (int z = lane; z < nz; z += 64)
      bctr[((size_t)b * nblocks + u / UB) * nz + z] = 0;
  const int32_t* mb = meta + (size_t)b * nunits * 4;
  // Lane j loads the whole record of unit u + j (one 16-byte load): lane 0
  // gives the tail, lanes 1.. the continuation flags and head lengths of the
  // units after u, so the common case needs no further metadata round trip.
  const int vj = u + lane;
  const int4 mv = vj < nunits ? reinterpret_cast<const int4*>(mb)[vj]
                              : int4{0, 0, 0, 0};
  static_assert(UnitMeta::TAIL_ID == 0 && UnitMeta::TAIL_LEN == 1 &&
                    UnitMeta::HEAD_LEN == 2 && UnitMeta::THROUGH == 3,
                "int4 view of the unit record");
  const int tail_len = __builtin_amdgcn_readfirstlane(mv.y);
  if (tail_len == 0) return;
  const int id = __builtin_amdgcn_readfirstlane(mv.x);
  if ((uint32_t)id >= (uint32_t)K) return;
  const int32_t* bmb = bmeta + (size_t)b * nblocks * 2;

  // The run continues through units u+1 .. e (e = first unit after u that
  // is not wholly inside the run; the last unit never is, so e exists).
  // Items, in order: heads of units u+1 .. min(e, end of u's block), then
  // full blocks, then heads of the units of the block holding e.  Units
  // u+1 .. bend-1 are lanes 1 .. bend-1-u (at most 63).
  const int bend = min((u / UB + 1) * UB, nunits);
  int n1, nblk = 0, n3 = 0, beta0 = u / UB + 1, v3 = 0;
  bool simple = false;  // the run ends inside u's block: lengths from mv
  {
    const bool stop = lane >= 1 && vj < bend && mv.w == 0;
    const uint64_t m = __builtin_amdgcn_ballot_w64(stop);
    if (m) {
      n1 = __builtin_ctzll(m);  // units u+1 .. u+n1 (lanes 1 .. n1)
      simple = true;
    } else {
      n1 = bend - (u + 1);
      int be = -1;
      for (int b0 = beta0; be < 0 && b0 < nblocks; b0 += 64) {
        const int bb = b0 + lane;
        const bool nf = bb < nblocks && bmb[(size_t)bb * 2] != tag;
        const uint64_t mm = __builtin_amdgcn_ballot_w64(nf);
        if (mm) be = b0 + (int)__builtin_ctzll(mm);
      }
      if (be < 0) be = nblocks - 1;  // unreachable: the last block is not full
      nblk = be - beta0;
      v3 = be * UB;
      const int w = v3 + lane;
      const bool st = w < nunits && mb[(size_t)w * 4 + UnitMeta::THROUGH] == 0;
      const uint64_t m3 = __builtin_amdgcn_ballot_w64(st);
      n3 = m3 ? (int)__builtin_ctzll(m3) + 1 : min(UB, nunits - v3);
    }
  }
  const int n = n1 + nblk + n3;
  const float* pb = part + (size_t)b * nunits * 2 * D;
  const float* bp = bpart + (size_t)b * nblocks * D;
  auto row = [&](int i) -> const float* {
    if (i < n1) return pb + ((size_t)(u + 1 + i) * 2 + 0) * D;
    if (i < n1 + nblk) return bp + (size_t)(beta0 + i - n1) * D;
    return pb + ((size_t)(v3 + i - n1 - nblk) * 2 + 0) * D;
  };
  // Row count: lanes over items, then a wave sum (integer, order-free).
  int l = simple ? (lane >= 1 && lane <= n1 ? mv.z : 0) : 0;
  for (int i = simple ? n : lane; i < n; i += 64) {
    if (i < n1)
      l += mb[(size_t)(u + 1 + i) * 4 + UnitMeta::HEAD_LEN];
    else if (i < n1 + nblk)
      l += bmb[(size_t)(beta0 + i - n1) * 2 + 1];
    else
      l += mb[(size_t)(v3 + i - n1 - nblk) * 4 + UnitMeta::HEAD_LEN];
  }
  const int len = tail_len + wave_sum_i(l);

  const bool fused = fin.cent != nullptr;  // uniform
  float* dst = fused ? fin_row[wave] : sums + ((size_t)b * K + id) * D;
  const float* tail = pb + ((size_t)u * 2 + 1) * D;
  const int add = (overwrite || fused) ? 0 : 1;
  if (D % 4 == 0)
    wave_ordered_sum<4>(tail, n, 0, D, row, dst, add, lane);
  else
    wave_ordered_sum<1>(tail, n, 0, D, row, dst, add, lane);
  if (fused) {
    wave_lds_sync();
    finalize_row<DT>(fin_row[wave], len, fin.cent + ((size_t)b * K + id) * D,
                     fin.c_sq + (size_t)b * K + id, fin.shift, D, lane);
    return;
  }
  if (lane == 0) {
    int32_t* cp = counts + (size_t)b * K + id;
    if (overwrite)
      *cp = len;
    else
      atomicAdd(cp, len);
  }
}

// ---------------------------------------------------------------------------
// Sort-free update of the Lloyd loop for short rows (update_scan).
//
// With N <= SCAN_NMAX points per row the loop replaces its three launches
// after the assign (label sort, update_runs, update_merge) by one.  Each
// workgroup owns `kpw` consecutive labels of one batch row.  It reads the
// whole row of labels into registers, counting the labels below its first
// one (the start of its range of sorted positions), and sets bit i of
// owned label j's bitmap for each owned point i.  The stable sort's order
// is label-major, index-minor, so the set bits of the concatenated bitmaps
// are its rows in sorted order: an exclusive scan of popcounts gives every
// owned row its sorted position without sorting anything else, and the row's
// point index is written to LDS there (a window of SCAN_CAP positions at a
// time).  From there the sums follow the sort path's units and order bit
// for bit: sorted positions are cut into units of `ur` rows (choose_ur),
// each piece of a run inside one unit is summed row by row in sorted order
// from zero, a run inside one unit is finalized at once, and a longer run
// keeps its tail partial (first unit) and head partials (later units) in
// the update workspace, then sums full 64-unit blocks and the run itself by
// wave_ordered_sum in update_merge's item order (tail, heads of the start
// block, block partials, heads of the end block), so the centroids, c_sq
// and shift equal those of label_sort + update_runs + update_merge.
// Every workgroup reads the whole row of labels and a label's rows are
// summed by its owner alone, so the route serves short rows only.
// FKC_SCAN_ONE=0 (compile time, for A/B builds) sends one-label
// workgroups through the bitmap placement too.
#ifndef FKC_SCAN_ONE
#define FKC_SCAN_ONE 1
#endif
constexpr int SCAN_NMAX = 32768;   // labels of a row, at most
constexpr int SCAN_KPW = 16;       // labels owned per workgroup, at most
constexpr int SCAN_CAP = 16384;    // sorted positions per placement window
constexpr int SCAN_T = 1024;       // threads per workgroup (16 waves)
constexpr int SCAN_W = SCAN_T / 64;
constexpr int SCAN_UMAX = SCAN_NMAX / (4 * SCAN_T);  // label quads per thread
constexpr int SCAN_BM = SCAN_KPW * SCAN_NMAX / 32;   // bitmap words (64 KB)

// SCAN_U: label quads per thread (N <= 4 * SCAN_T * SCAN_U).  ONE: the
// workgroup owns one label (kpw == 1).  Its rows are then placed without
// bitmaps: each lane keeps a mask of its owned slots and the owned counts
// of its quads, packed three to a word, so a few DPP scans rank every
// 256-point chunk (one wave's labels of one quad index u); the chunk totals
// are scanned once in chunk order (which is index order), and each lane
// loops over its own set bits only: a row's sorted position is its chunk's
// offset plus the owned rows of lower lanes and of its own lower slots.
// The bitmap's LDS then holds the run's unit partials when they fit (a run
// over a few units), which wave 0 merges straight into the finalize.  The
// kernel issues the same instructions on 16 waves per CU, so it is bound by
// their count: this form avoids the bitmap walk's per-word loops and
// branches.  Positions, pieces and summation order are those of the bitmap
// path, so the bits are the same.
template <int DT, int VEC, int NI, int SCAN_U, bool ONE>
__global__ void __launch_bounds__(SCAN_T)
update_scan_kernel(const typename Elem<DT>::T* __restrict__ x,
                   const int32_t* __restrict__ ids, float* __restrict__ part,
                   float* __restrict__ bpart, int N, int K, int D, int nunits,
                   int nblocks, int ur, int kpw, int vec4,
                   FinArgs<typename Elem<DT>::T> fin,
                   const int32_t* __restrict__ ctrl) {
  using T = typename Elem<DT>::T;
  using RC = RawCols<DT, VEC>;
  using R = typename RC::T;
  // Sorted positions of the current window; ONE: 128 more entries give
  // each lane a slot of its own for the stores of rows it does not place.
  __shared__ uint16_t s_perm[SCAN_CAP + (ONE ? 128 : 0)];
  __shared__ float s_row[SCAN_W][FIN_DMAX];
  // Bit i of word w of label j's bitmap (words j * wpl .. j * wpl + wpl - 1)
  // is set when point 32 w + i has label k0 + j.  ONE: unit partials.
  __shared__ __attribute__((aligned(16))) uint32_t s_bm[SCAN_BM];
  __shared__ int s_off[SCAN_KPW + 1];
  __shared__ int s_red[SCAN_W];
  __shared__ int s_cnt[ONE ? SCAN_W * SCAN_U : 1];  // ONE: matches per chunk
  if (loop_done(ctrl)) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = blockIdx.y;
  const int k0 = blockIdx.x * kpw;
  const int nk = ONE ? 1 : min(kpw, K - k0);  // >= 1: the grid covers K exactly
  const int32_t* ib = ids + (size_t)b * N;
  const T* xb = x + (size_t)b * N * D;
  float* partb = part + (size_t)b * nunits * 2 * D;
  float* bpartb = bpart + (size_t)b * nblocks * D;
  const int wpl = (N + 31) / 32;  // bitmap words per owned label
  const int nbw = nk * wpl;       // <= SCAN_BM (plan)
  if constexpr (!ONE)
    for (int i = tid; i < nbw; i += SCAN_T) s_bm[i] = 0u;

  // 1. The row's labels stay in registers: thread t holds labels
  // 4 (t + SCAN_T u) + c, u < SCAN_U, c < 4.  All loads are in flight
  // before any is used.  Branch-free: indices are clamped into the row and
  // labels past N read as INT_MAX (never owned, never below k0).  vec4
  // implies N % 4 == 0, so a quad is wholly inside the row or wholly past it.
  int lab[SCAN_U][4];
  if (vec4) {
#pragma unroll
    for (int u = 0; u < SCAN_U; ++u) {
      const int i0 = 4 * (tid + SCAN_T * u);
      const int4 v = *reinterpret_cast<const int4*>(ib + min(i0, N - 4));
      const bool in = i0 < N;
      lab[u][0] = in ? v.x : INT_MAX;
      lab[u][1] = in ? v.y : INT_MAX;
      lab[u][2] = in ? v.z : INT_MAX;
      lab[u][3] = in ? v.w : INT_MAX;
    }
  } else {
#pragma unroll
    for (int u = 0; u < SCAN_U; ++u)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int i = 4 * (tid + SCAN_T * u) + c;
        const int l = ib[min(i, N - 1)];
        lab[u][c] = i < N ? l : INT_MAX;
      }
  }
  int below = 0;
#pragma unroll
  for (int u = 0; u < SCAN_U; ++u)
#pragma unroll
    for (int c = 0; c < 4; ++c) below += (unsigned)lab[u][c] < (unsigned)k0 ? 1 : 0;
  below = __builtin_amdgcn_readlane(wave_incl_scan(below), 63);
  if (lane == 0) s_red[wave] = below;
  // ONE: chunk (u, wave) holds points 4 (SCAN_T u + 64 wave) .. + 255, so
  // chunk q = SCAN_W u + wave runs in index order; rk[u] is this lane's
  // first match's rank inside its chunk (the matches of lower lanes).  The
  // lanes' match counts of three quads share a word (10-bit fields: a
  // chunk holds at most 256), so one DPP scan ranks three chunks.
  // own: bit 4u + c set when label (u, c) is the owned one (built from the
  // last slot down, one shift-and-add per label).
  int rk[ONE ? SCAN_U : 1];
  uint32_t own = 0u;
  if constexpr (ONE) {
#pragma unroll
    for (int u = SCAN_U - 1; u >= 0; --u)
#pragma unroll
      for (int c = 3; c >= 0; --c) own = own + own + (lab[u][c] == k0 ? 1u : 0u);
    constexpr int NW = (SCAN_U + 2) / 3;
    int pk[NW];
#pragma unroll
    for (int w = 0; w < NW; ++w) pk[w] = 0;
#pragma unroll
    for (int u = 0; u < SCAN_U; ++u)
      pk[u / 3] += __builtin_popcount((own >> (4 * u)) & 15u) << (10 * (u % 3));
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const int inc = wave_incl_scan(pk[w]);
      const int exc = inc - pk[w];
      const int tot = __builtin_amdgcn_readlane(inc, 63);
#pragma unroll
      for (int f = 0; f < 3 && 3 * w + f < SCAN_U; ++f) {
        const int u = 3 * w + f;
        rk[u] = (exc >> (10 * f)) & 1023;
        if (lane == 0) s_cnt[SCAN_W * u + wave] = (tot >> (10 * f)) & 1023;
      }
    }
  }
  __syncthreads();  // bitmaps cleared, s_red (and s_cnt) written
  int S0 = 0;
#pragma unroll
  for (int w = 0; w < SCAN_W; ++w) S0 += s_red[w];

  int first = 0, w_lo = 0, w_hi = 0, S1;
  if constexpr (ONE) {
    // Exclusive offsets of the SCAN_W * SCAN_U chunks: lane l scans chunks
    // 2l and 2l + 1 as a pair; chunk q's offset is then the pair offset of
    // lane q / 2, plus chunk q - 1 when q is odd (q's parity is the wave's).
    constexpr int NC = SCAN_W * SCAN_U;  // <= 128
    const int ca = 2 * lane < NC ? s_cnt[2 * lane] : 0;
    const int cb = 2 * lane + 1 < NC ? s_cnt[2 * lane + 1] : 0;
    const int inc = wave_incl_scan(ca + cb);
    const int exc = inc - ca - cb;
#pragma unroll
    for (int u = 0; u < SCAN_U; ++u) {
      const int q = SCAN_W * u + wave;
      int o = __builtin_amdgcn_readlane(exc, q >> 1);
      if (q & 1) o += __builtin_amdgcn_readlane(ca, q >> 1);
      rk[u] += S0 + o;
    }
    S1 = S0 + __builtin_amdgcn_readlane(inc, 63);
    if (tid == 0) {
      s_off[0] = S0;
      s_off[1] = S1;
    }
  } else {
    // 2. Each owned row sets its bit.
#pragma unroll
    for (int u = 0; u < SCAN_U; ++u)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const unsigned j = (unsigned)(lab[u][c] - k0);
        if (j < (unsigned)nk) {
          const int i = 4 * (tid + SCAN_T * u) + c;
          atomicOr(&s_bm[j * wpl + (i >> 5)], 1u << (i & 31));
        }
      }
    __syncthreads();

    // 3. In label-major, index-minor order (the stable sort's order) the set
    // bits of the concatenated bitmaps are the owned rows, so a row's sorted
    // position is S0 plus the set bits before it.  Thread t takes words
    // t * wpt .. t * wpt + wpt - 1; an exclusive scan of the threads' counts
    // gives each thread its first position.
    const int wpt = (nbw + SCAN_T - 1) / SCAN_T;  // <= SCAN_BM / SCAN_T
    w_lo = min(tid * wpt, nbw);
    w_hi = min(w_lo + wpt, nbw);
    int mine = 0;
    for (int w = w_lo; w < w_hi; ++w) mine += __builtin_popcount(s_bm[w]);
    int incl = mine;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(incl, d, 64);
      if (lane >= d) incl += y;
    }
    __syncthreads();  // s_red (S0's inputs) read by every thread
    if (lane == 63) s_red[wave] = incl;
    __syncthreads();
    first = S0 + incl - mine;
    for (int w = 0; w < wave; ++w) first += s_red[w];
    // A label's first position: the thread holding its first word.
    {
      int p = first;
      for (int w = w_lo; w < w_hi; ++w) {
        if (w % wpl == 0) s_off[w / wpl] = p;
        p += __builtin_popcount(s_bm[w]);
      }
      if (tid == SCAN_T - 1) s_off[nk] = p;
    }
    __syncthreads();
    S1 = s_off[nk];
  }
  if (S1 == S0) return;  // every owned label is empty: its centroid stands

  int col[NI];
  bool cok[NI];
  int lcol[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    col[i] = (lane + 64 * i) * VEC;
    cok[i] = col[i] < D;
    lcol[i] = cok[i] ? col[i] : 0;
  }
  using Acc = float[NI][VEC];
  // Rows in flight per wave: 32 raw words, 16 where a raw load is 8 bytes
  // (fp32 pairs), so the gather fits beside the labels in 128 registers.
  constexpr int RB = (sizeof(R) >= 8 ? 16 : 32) / NI;

  // Finalize label k0 + j from a row of sums in this wave's LDS row.
  auto finish = [&](int j, int cnt) {
    wave_lds_sync();
    const int id = k0 + j;
    finalize_row<DT>(s_row[wave], cnt, fin.cent + ((size_t)b * K + id) * D,
                     fin.c_sq + (size_t)b * K + id, fin.shift, D, lane);
    wave_lds_sync();
  };

  // The items of a run over several units, in update_merge's order: the
  // heads of units us+1 .. bend-1 (n1), then nblk full 64-unit blocks from
  // block beta0 (their block partials), then the heads of units v3 .. ue
  // (n3); the tail of unit us comes first.
  auto run_items = [&](int s, int e, int& n1, int& beta0, int& nblk, int& v3,
                       int& n3) {
    const int us = s / ur, ue = (e - 1) / ur;
    const int bend = min((us / UB + 1) * UB, nunits);
    beta0 = us / UB + 1;
    nblk = 0;
    n3 = 0;
    v3 = 0;
    if (ue < bend) {
      n1 = ue - us;
      return;
    }
    n1 = bend - (us + 1);
    int be = beta0;
    while ((int64_t)(be + 1) * UB * ur < e) ++be;  // blocks wholly inside
    nblk = be - beta0;
    v3 = be * UB;
    n3 = ue - v3 + 1;
  };
  // ONE: a run over 2+ units and no full block keeps its unit partials in
  // LDS (slot u - us holds unit u's piece: slot 0 the tail, then the heads
  // in item order) when they fit where the bitmaps would be.
  float* s_part = reinterpret_cast<float*>(s_bm);
  bool lds_part = false;
  if constexpr (ONE) {
    const int us = S0 / ur, ue = (S1 - 1) / ur;
    if (us != ue) {
      int n1, beta0, nblk, v3, n3;
      run_items(S0, S1, n1, beta0, nblk, v3, n3);
      lds_part = nblk == 0 && (ue - us + 1) * D <= SCAN_BM;
    }
  }

  // 4. Windows of SCAN_CAP sorted positions, starting at a unit boundary:
  // each thread writes the point index of each of its owned rows whose
  // position falls in the window, then the window's pieces (a run's rows
  // inside one unit) are summed, spread over the waves.  A run inside one
  // unit is finalized at once; a longer run's pieces go to the workspace
  // (ONE: to LDS where lds_part).
  for (int W0 = S0 / ur * ur; W0 < S1; W0 += SCAN_CAP) {
    const int W1 = min(W0 + SCAN_CAP, S1);
    if constexpr (ONE) {
      // One trip per owned row of the lane (owned rows are sparse): its
      // quad's rank rk[u] picked by selects, plus the owned rows below it
      // in the same quad; a row outside the window stores into the lane's
      // own spare entry.
      const unsigned span = (unsigned)(W1 - W0);
      for (uint32_t m = own; m != 0u; m &= m - 1u) {
        const int bit = __builtin_ctz(m);
        const int u = bit >> 2;
        int r = rk[0];
#pragma unroll
        for (int v = 1; v < SCAN_U; ++v) r = u == v ? rk[v] : r;
        const int p = r + __builtin_popcount(own & (((1u << bit) - 1u) & (15u << (4 * u)))) - W0;
        s_perm[(unsigned)p < span ? p : SCAN_CAP + 2 * lane] =
            (uint16_t)(4 * (tid + SCAN_T * u) + (bit & 3));
      }
    } else if (first < W1) {
      int p = first;
      for (int w = w_lo; w < w_hi && p < W1; ++w) {
        uint32_t m = s_bm[w];
        const int i0 = (w % wpl) * 32;
        while (m != 0u) {
          const int bit = __builtin_ctz(m);
          m &= m - 1u;
          if (p >= W0 && p < W1) s_perm[p - W0] = (uint16_t)(i0 + bit);
          ++p;
        }
      }
    }
    __syncthreads();
    // Pieces in label-major order, (label j, unit u) for the units of
    // label j's rows inside the window; piece q goes to wave q % SCAN_W.
    const int uw0 = W0 / ur, uw1 = (W1 - 1) / ur;  // the window's units
    for (int q = wave;; q += SCAN_W) {
      int j = 0, u = 0, qq = q;
      for (; j < nk; ++j) {
        const int s = s_off[j], e = s_off[j + 1];
        if (s == e) continue;
        const int lo = max(s / ur, uw0), hi = min((e - 1) / ur, uw1);
        const int np = hi >= lo ? hi - lo + 1 : 0;
        if (qq < np) {
          u = lo + qq;
          break;
        }
        qq -= np;
      }
      if (j >= nk) break;
      {
        const int s = s_off[j], e = s_off[j + 1];
        const int a = max(max(u * ur, s), W0), z = min(min((u + 1) * ur, e), W1);
        Acc acc;
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
          for (int v = 0; v < VEC; ++v) acc[i][v] = 0.f;
        for (int r0 = a; r0 < z; r0 += RB) {
          // The batch's point indices, one per lane in a single LDS read,
          // then taken lane by lane (no LDS round trip per row); min keeps a
          // row index inside the batch row whatever LDS holds.
          const int lidx = min((int)s_perm[min(r0 + lane, z - 1) - W0], N - 1);
          R raw[RB][NI];
#pragma unroll
          for (int jj = 0; jj < RB; ++jj) {
            const int idx = __builtin_amdgcn_readlane(lidx, jj);
            const T* row = xb + (size_t)idx * D;
#pragma unroll
            for (int i = 0; i < NI; ++i) raw[jj][i] = RC::load(row + lcol[i]);
          }
#pragma unroll
          for (int jj = 0; jj < RB; ++jj) {
            if (r0 + jj < z) {
#pragma unroll
              for (int i = 0; i < NI; ++i) {
                float f[VEC];
                RC::cvt(raw[jj][i], f);
#pragma unroll
                for (int v = 0; v < VEC; ++v) acc[i][v] = acc[i][v] + f[v];
              }
            }
          }
        }
        const int us = s / ur, ue = (e - 1) / ur;
        float* dst = us == ue  ? s_row[wave]
                     : lds_part ? s_part + (size_t)(u - us) * D
                                : partb + ((size_t)u * 2 + (u == us ? 1 : 0)) * D;
#pragma unroll
        for (int i = 0; i < NI; ++i)
          if (cok[i]) {
#pragma unroll
            for (int v = 0; v < VEC; ++v) dst[col[i] + v] = acc[i][v];
          }
        if (us == ue) finish(j, e - s);
      }
    }
    __syncthreads();
  }

  // ONE with the partials in LDS: no blocks, one run; wave 0 merges and
  // finalizes it.
  if constexpr (ONE) {
    if (lds_part) {
      if (wave == 0)
        merge_finalize<DT>(s_part, (S1 - 1) / ur - S0 / ur, S1 - S0,
                           fin.cent + ((size_t)b * K + k0) * D,
                           fin.c_sq + (size_t)b * K + k0, fin.shift, D, lane);
      return;
    }
  }

  // 5. Runs over several units: full 64-unit blocks first (update_runs'
  // block sums), then each run in update_merge's item order.
  // The full blocks of all owned runs, in label order, spread over the
  // waves (a crowded label's blocks are summed in parallel).
  for (int q = wave;; q += SCAN_W) {
    int beta = -1, qq = q;
    for (int j = 0; j < nk; ++j) {
      const int s = s_off[j], e = s_off[j + 1];
      if (e - s == 0 || s / ur == (e - 1) / ur) continue;
      int n1, beta0, nblk, v3, n3;
      run_items(s, e, n1, beta0, nblk, v3, n3);
      if (qq < nblk) {
        beta = beta0 + qq;
        break;
      }
      qq -= nblk;
    }
    if (beta < 0) break;
    auto row = [&](int i) {
      return partb + ((size_t)(beta * UB + i) * 2 + 0) * D;
    };
    float* dst = bpartb + (size_t)beta * D;
    if (D % 4 == 0)
      wave_ordered_sum<4>(nullptr, UB, 0, D, row, dst, 0, lane);
    else
      wave_ordered_sum<1>(nullptr, UB, 0, D, row, dst, 0, lane);
  }
  __syncthreads();
  for (int j = wave; j < nk; j += SCAN_W) {
    const int s = s_off[j], e = s_off[j + 1];
    if (e - s == 0 || s / ur == (e - 1) / ur) continue;
    int n1, beta0, nblk, v3, n3;
    run_items(s, e, n1, beta0, nblk, v3, n3);
    const int us = s / ur;
    auto row = [&](int i) -> const float* {
      if (i < n1) return partb + ((size_t)(us + 1 + i) * 2 + 0) * D;
      if (i < n1 + nblk) return bpartb + (size_t)(beta0 + i - n1) * D;
      return partb + ((size_t)(v3 + i - n1 - nblk) * 2 + 0) * D;
    };
    const float* tail = partb + ((size_t)us * 2 + 1) * D;
    const int n = n1 + nblk + n3;
    if (D % 4 == 0)
      wave_ordered_sum<4>(tail, n, 0, D, row, s_row[wave], 0, lane);
    else
      wave_ordered_sum<1>(tail, n, 0, D, row, s_row[wave], 0, lane);
    finish(j, e - s);
  }
}

// Column slices per lane pass: VEC columns per lane (2 when D is even), NI
// slices of 64 lanes per row (1, 2 or 4), and grid.z column blocks beyond.
inline int runs_vec(int64_t D) { return row_vec((int)D); }
inline int runs_ni(int64_t D) {
  const int64_t slices = (D + 64 * runs_vec(D) - 1) / (64 * runs_vec(D));
  return slices <= 1 ? 1 : (slices <= 2 ? 2 : 4);
}
inline int64_t runs_zblocks(int64_t D) {
  const int64_t cols = 64 * runs_vec(D) * runs_ni(D);
  return (D + cols - 1) / cols;
}

// Workspace layout, shared by the size query and the launcher.  bmeta and
// bctr are consecutive: the control region the Lloyd loop clears once.
struct UpdateBufs {
  float* part;      // [B][nunits][2][D] unit head / tail partials
  int32_t* meta;    // [B][nunits][4] unit records
  float* bpart;     // [B][nblocks][D] block partials
  int32_t* bmeta;   // [B][nblocks][2] block flag, row count
  int32_t* bctr;    // [B][nblocks][nz] arrival counters
  int64_t nunits, nblocks, nz;
  int64_t nctl;     // int32 words from bmeta to the end of bctr
  size_t used;
};

UpdateBufs carve_update(void* ws, int64_t B, int64_t N, int64_t D) {
  const int ur = choose_ur(B, N);
  UpdateBufs w{};
  w.nunits = (N + ur - 1) / ur;
  w.nblocks = (w.nunits + UB - 1) / UB;
  w.nz = runs_zblocks(D);
  Carve c(ws);
  w.part = c.take<float>((size_t)B * w.nunits * 2 * D);
  w.meta = c.take<int32_t>((size_t)B * w.nunits * 4);
  w.bpart = c.take<float>((size_t)B * w.nblocks * D);
  const size_t ctl0 = c.used;
  w.bmeta = c.take<int32_t>((size_t)B * w.nblocks * 2);
  w.bctr = c.take<int32_t>((size_t)B * w.nblocks * w.nz);
  w.nctl = (int64_t)((c.used - ctl0) / sizeof(int32_t));
  w.used = c.used;
  return w;
}

template <int DT, int VEC, int NI, bool INDEXED>
int launch_runs_t(const void* x, const int32_t* perm, const int32_t* sids,
                  float* sums, int32_t* counts, const UpdateBufs& w, int64_t B,
                  int64_t N, int64_t K, int64_t D, bool overwrite,
                  const BlockArgs& blk, FinArgs<typename Elem<DT>::T> fin,
                  const int32_t* ctrl, hipStream_t s) {
  using T = typename Elem<DT>::T;
  const int ur = choose_ur(B, N);
  dim3 grid((unsigned)((w.nunits + 3) / 4), (unsigned)B, (unsigned)w.nz);
  hipLaunchKernelGGL((update_runs_kernel<DT, VEC, NI, INDEXED>), grid,
                     dim3(UT), 0, s, static_cast<const T*>(x), perm, sids,
                     sums, counts, w.part, w.meta, (int)N, (int)K, (int)D,
                     (int)w.nunits, ur, overwrite ? 1 : 0, blk, fin, ctrl);
  return check_launch("update_runs");
}

template <int DT, bool INDEXED>
int launch_runs_dt(const void* x, const int32_t* perm, const int32_t* sids,
                   float* sums, int32_t* counts, const UpdateBufs& w,
                   int64_t B, int64_t N, int64_t K, int64_t D, bool overwrite,
                   const BlockArgs& blk, FinArgs<typename Elem<DT>::T> fin,
                   const int32_t* ctrl, hipStream_t s) {
#define FKC_RUNS(V, NI_)                                                     \
  return launch_runs_t<DT, V, NI_, INDEXED>(x, perm, sids, sums, counts, w, \
                                            B, N, K, D, overwrite, blk, fin, \
                                            ctrl, s)
  const int vec = runs_vec(D), ni = runs_ni(D);
  if (vec == 2) {
    if (ni == 1) FKC_RUNS(2, 1);
    if (ni == 2) FKC_RUNS(2, 2);
    FKC_RUNS(2, 4);
  }
  if (ni == 1) FKC_RUNS(1, 1);
  if (ni == 2) FKC_RUNS(1, 2);
  FKC_RUNS(1, 4);
#undef FKC_RUNS
}

template <int DT>
int launch_update_t(const void* x, const int32_t* perm,
                    const int32_t* ids_sorted, float* sums, int32_t* counts,
                    const UpdateBufs& w, int64_t B, int64_t N, int64_t K,
                    int64_t D, bool overwrite, int64_t seq,
                    FinArgs<typename Elem<DT>::T> fin, const int32_t* ctrl,
                    hipStream_t s) {
  // With one block every run ends inside it and block partials are unused.
  // The Lloyd loop (seq >= 0) sums full blocks inside update_runs, its flags
  // tagged with the call's number; otherwise update_blocks does, tag 1.
  const bool in_runs = seq >= 0 && w.nblocks > 1;
  BlockArgs blk{w.bpart, w.bmeta, in_runs ? w.bctr : nullptr, (int)w.nblocks,
                in_runs ? (int)(1 + seq % (INT_MAX - 1)) : 1};
  int rc = perm != nullptr
               ? launch_runs_dt<DT, true>(x, perm, ids_sorted, sums, counts, w,
                                          B, N, K, D, overwrite, blk, fin,
                                          ctrl, s)
               : launch_runs_dt<DT, false>(x, perm, ids_sorted, sums, counts,
                                           w, B, N, K, D, overwrite, blk, fin,
                                           ctrl, s);
  if (rc) return rc;
  if (w.nblocks > 1 && !in_runs) {
    dim3 bgrid((unsigned)((w.nblocks + 3) / 4), (unsigned)B);
    hipLaunchKernelGGL(update_blocks_kernel, bgrid, dim3(UT), 0, s, w.part,
                       w.meta, w.bpart, w.bmeta, (int)D, (int)w.nunits,
                       (int)w.nblocks, blk.tag, ctrl);
    rc = check_launch("update_blocks");
    if (rc) return rc;
  }
  dim3 grid((unsigned)((w.nunits + 3) / 4), (unsigned)B);
  hipLaunchKernelGGL((update_merge_kernel<DT>), grid, dim3(UT), 0, s, w.part,
                     w.meta, w.bpart, w.bmeta, sums, counts, (int)K, (int)D,
                     (int)w.nunits, (int)w.nblocks, overwrite ? 1 : 0, blk.tag,
                     blk.ctr, (int)w.nz, fin, ctrl);
  return check_launch("update_merge");
}

template <int DT, int VEC, int NI>
int launch_scan_t(const void* x, const int32_t* ids, const UpdateBufs& w,
                  int64_t B, int64_t N, int64_t K, int64_t D, int kpw,
                  int vec4, const UpdateFinalize& f, const int32_t* ctrl,
                  hipStream_t s) {
  using T = typename Elem<DT>::T;
  FinArgs<T> fa{static_cast<T*>(f.cent), f.c_sq, f.shift};
  dim3 grid((unsigned)((K + kpw - 1) / kpw), (unsigned)B);
  // Two register budgets for the row's labels: rows up to 8192 hold two
  // quads per thread, longer ones SCAN_UMAX; one owned label per workgroup
  // takes the ballot placement.
#define FKC_SCAN_LAUNCH(U, ONE_)                                              \
  hipLaunchKernelGGL((update_scan_kernel<DT, VEC, NI, U, ONE_>), grid,        \
                     dim3(SCAN_T), 0, s, static_cast<const T*>(x), ids,       \
                     w.part, w.bpart, (int)N, (int)K, (int)D, (int)w.nunits,  \
                     (int)w.nblocks, choose_ur(B, N), kpw, vec4, fa, ctrl)
  const bool one = FKC_SCAN_ONE && kpw == 1;
  if (N <= 8 * SCAN_T) {
    if (one)
      FKC_SCAN_LAUNCH(2, true);
    else
      FKC_SCAN_LAUNCH(2, false);
  } else {
    if (one)
      FKC_SCAN_LAUNCH(SCAN_UMAX, true);
    else
      FKC_SCAN_LAUNCH(SCAN_UMAX, false);
  }
#undef FKC_SCAN_LAUNCH
  return check_launch("update_scan");
}

template <int DT>
int launch_scan_dt(const void* x, const int32_t* ids, const UpdateBufs& w,
                   int64_t B, int64_t N, int64_t K, int64_t D, int kpw,
                   int vec4, const UpdateFinalize& f, const int32_t* ctrl,
                   hipStream_t s) {
#define FKC_SCAN(V, NI_) \
  return launch_scan_t<DT, V, NI_>(x, ids, w, B, N, K, D, kpw, vec4, f, ctrl, s)
  const int vec = runs_vec(D), ni = runs_ni(D);
  if (vec == 2) {
    if (ni == 1) FKC_SCAN(2, 1);
    if (ni == 2) FKC_SCAN(2, 2);
    FKC_SCAN(2, 4);
  }
  if (ni == 1) FKC_SCAN(1, 1);
  if (ni == 2) FKC_SCAN(1, 2);
  FKC_SCAN(1, 4);
#undef FKC_SCAN
}

// Labels per workgroup of update_scan: the row's K labels spread so that
// the launch has about one workgroup per compute unit.
int64_t scan_kpw(int64_t B, int64_t K) {
  const int64_t o = scan_wgs_override();
  const int64_t w = o > 0 ? o : device_shape().cus;
  return (B * K + w - 1) / w;
}

}  // namespace

size_t update_workspace_bytes(int64_t B, int64_t N, int64_t D) {
  return carve_update(nullptr, B, N, D).used;
}

void update_control_region(void* ws, int64_t B, int64_t N, int64_t D,
                           int32_t** p, int64_t* n) {
  *p = nullptr;
  *n = 0;
  if (B == 0 || N == 0) return;
  const UpdateBufs w = carve_update(ws, B, N, D);
  *p = w.bmeta;
  *n = w.nctl;
}

int launch_update(const void* x, const int32_t* perm,
                  const int32_t* ids_sorted, float* sums, int32_t* counts,
                  int64_t B, int64_t N, int64_t K, int64_t D, int dtype,
                  bool overwrite, void* ws, size_t ws_bytes,
                  const int32_t* ctrl, hipStream_t s, const UpdateFinalize* fin,
                  bool* fused, int64_t seq) {
  if (fused) *fused = false;
  if (B == 0) return FKC_OK;
  if (N == 0) {
    if (!overwrite) return FKC_OK;
    int rc = launch_fill_f32(sums, 0.f, B * K * D, s);
    return rc ? rc : launch_fill_i32(counts, 0, B * K, s);
  }
  const size_t need = update_workspace_bytes(B, N, D);
  if (ws_bytes < need || ws == nullptr)
    return fail(FKC_ERR_WORKSPACE, "centroid_update: workspace %zu < %zu bytes",
                ws_bytes, need);
  if (reinterpret_cast<uintptr_t>(ws) % kWorkspaceAlign != 0)
    return fail(FKC_ERR_WORKSPACE,
                "centroid_update: workspace not %d-byte aligned",
                kWorkspaceAlign);
  if (seq >= 0 && !overwrite)
    return fail(FKC_ERR_INVALID, "centroid_update: a sequenced call overwrites");
  const UpdateBufs w = carve_update(ws, B, N, D);
  // Finalize fuses when a whole row fits one wave's column slices and LDS
  // row buffer (D <= 512; then grid.z == 1) and every label is valid.
  const bool fuse = fin != nullptr && fin->cent != nullptr && overwrite &&
                    D <= FIN_DMAX &&
                    D <= (int64_t)64 * runs_vec(D) * runs_ni(D);
  if (fused) *fused = fuse;
  switch (dtype) {
    case FKC_F32: {
      FinArgs<float> f{fuse ? static_cast<float*>(fin->cent) : nullptr,
                       fuse ? fin->c_sq : nullptr, fuse ? fin->shift : nullptr};
      return launch_update_t<FKC_F32>(x, perm, ids_sorted, sums, counts, w, B,
                                      N, K, D, overwrite, seq, f, ctrl, s);
    }
    case FKC_F16: {
      using T = typename Elem<FKC_F16>::T;
      FinArgs<T> f{fuse ? static_cast<T*>(fin->cent) : nullptr,
                   fuse ? fin->c_sq : nullptr, fuse ? fin->shift : nullptr};
      return launch_update_t<FKC_F16>(x, perm, ids_sorted, sums, counts, w, B,
                                      N, K, D, overwrite, seq, f, ctrl, s);
    }
    case FKC_BF16: {
      using T = typename Elem<FKC_BF16>::T;
      FinArgs<T> f{fuse ? static_cast<T*>(fin->cent) : nullptr,
                   fuse ? fin->c_sq : nullptr, fuse ? fin->shift : nullptr};
      return launch_update_t<FKC_BF16>(x, perm, ids_sorted, sums, counts, w, B,
                                       N, K, D, overwrite, seq, f, ctrl, s);
    }
    default:
      return fail(FKC_ERR_INVALID, "centroid_update: unknown dtype %d", dtype);
  }
}

bool update_scan_ok(int64_t B, int64_t N, int64_t K, int64_t D) {
  const int o = update_scan_override();
  if (o == 0) return false;
  if (B < 1 || N < 1 || N > SCAN_NMAX || K < 1 || K > 65535) return false;
  if (D < 1 || D > FIN_DMAX || D > (int64_t)64 * runs_vec(D) * runs_ni(D))
    return false;
  if (scan_kpw(B, K) > SCAN_KPW) return false;
  // Taken on its own for every row it can hold, where it measured faster
  // than the three launches it replaces (loop time per iteration, same box,
  // scan vs sort: c1's (1, 4096, 64, 128) f32 18.8 vs 24.8 us, c2's
  // (1, 32768, 256, 128) f16 mixture 27.1 vs 30.2, random rows
  // (1, 2048, 64, 128) 14.2 vs 20.6, (1, 8192, 256, 128) 17.4 vs 25.7,
  // (1, 8192, 1024, 64) bf16 21.9 vs 33.5, (4, 8192, 128, 64) 16.4 vs
  // 21.6, (1, 16384, 64, 32) 17.1 vs 20.0).  A label's rows are summed by
  // its owner's 16 waves alone, so rows crowded into one label cost more
  // than the sort path spreading them over the chip: half or 95% of 32768
  // points on one spot, 56-77 vs 34-41 us; at 16384 points 25.7 vs 30.8.
  return o == 1 || N <= 256 * K;
}

int launch_update_scan(const void* x, const int32_t* ids, int64_t B,
                       int64_t N, int64_t K, int64_t D, int dtype, void* ws,
                       size_t ws_bytes, const int32_t* ctrl, hipStream_t s,
                       const UpdateFinalize& fin) {
  if (!update_scan_ok(B, N, K, D))
    return fail(FKC_ERR_UNSUPPORTED, "update_scan: shape outside its plan");
  const size_t need = update_workspace_bytes(B, N, D);
  if (ws == nullptr || ws_bytes < need)
    return fail(FKC_ERR_WORKSPACE, "update_scan: workspace %zu < %zu bytes",
                ws_bytes, need);
  if (fin.cent == nullptr || fin.c_sq == nullptr)
    return fail(FKC_ERR_INVALID, "update_scan: no centroids to finalize");
  const UpdateBufs w = carve_update(ws, B, N, D);
  const int kpw = (int)scan_kpw(B, K);
  const int vec4 =
      (N % 4 == 0 && reinterpret_cast<uintptr_t>(ids) % 16 == 0) ? 1 : 0;
  switch (dtype) {
    case FKC_F32:
      return launch_scan_dt<FKC_F32>(x, ids, w, B, N, K, D, kpw, vec4, fin, ctrl, s);
    case FKC_F16:
      return launch_scan_dt<FKC_F16>(x, ids, w, B, N, K, D, kpw, vec4, fin, ctrl, s);
    case FKC_BF16:
      return launch_scan_dt<FKC_BF16>(x, ids, w, B, N, K, D, kpw, vec4, fin, ctrl, s);
    default:
      return fail(FKC_ERR_INVALID, "update_scan: unknown dtype %d", dtype);
  }
}

}  // namespace fkc
