// Stable LSD radix sort of cluster labels (replaces torch.sort at
// flash_kmeans_cuda/ops.py:89; the reference asks stable=False, this sort is
// stable so its permutation is reproducible bit for bit).
//
// Keys are labels in [0,K); a label outside that range sorts as K, i.e. after
// every valid label, keeping index order.  The key width is
// bits = ceil(log2(K+1)) so the sentinel has a bin, or ceil(log2(K)) when the
// caller vouches that every label is valid (labels straight from the assign
// kernel), split into passes of at most 8 bits.
// Each pass is reduce-then-scan, with no inter-workgroup waiting:
//   sort_hist    : per tile of 4096 keys (1024 for small N), a digit
//                  histogram in LDS, written digit-major to
//                  hist[b][digit][tile];
//   sort_scan    : exclusive scan of hist[b] (digit-major, so the scan gives
//                  every (digit, tile) its global output offset);
//   sort_scatter : each wave ranks its share of the tile (8 waves x 512
//                  keys, or 4 waves x 256 keys for 1024-key tiles) stably,
//                  64 keys at a time: a ballot per digit bit yields, for every lane, the
//                  mask of lanes holding the same digit ("multi-split"); its
//                  rank is the per-wave digit counter plus the matching lanes
//                  below it.  Keys are placed in LDS in tile-sorted order,
//                  then each digit's run is copied to its global slot, so the
//                  writes are runs of consecutive addresses.
// The carried payload is the original index; the last pass writes the
// user's sorted_ids / perm.
#include "device_util.hpp"
#include "fkc_internal.hpp"

namespace fkc {
namespace {

constexpr int HT = 256;           // threads of the histogram kernel

// Keys per tile (one workgroup of each kernel): 4096, or 1024 for small N so
// that the grid still has some width.
template <int TILE_>
struct Geom {
  static constexpr int TILE = TILE_;
  static constexpr int ST = TILE_ >= 4096 ? 512 : 256;  // scatter threads
  static constexpr int SW = ST / 64;                    // scatter waves
  static constexpr int PER_WAVE = TILE / SW;
  static constexpr int CHUNKS = PER_WAVE / 64;
  static_assert(ST >= 256 && CHUNKS >= 1, "scatter geometry");
};

__device__ inline uint32_t sort_key(int32_t id, int K) {
  return (uint32_t)id < (uint32_t)K ? (uint32_t)id : (uint32_t)K;
}

// Per-batch stride of the digit table: room for 256 digits x ntiles,
// rounded to whole int4s so every batch row starts 16-byte aligned.
inline int64_t table_stride(int64_t ntiles) { return (256 * ntiles + 3) / 4 * 4; }

template <int TILE>
__global__ void __launch_bounds__(HT)
sort_hist_kernel(const int32_t* __restrict__ keys, int32_t* __restrict__ hist,
                 int N, int K, int shift, int bits, int ntiles, int64_t hstride,
                 const int32_t* __restrict__ ctrl) {
  if (loop_done(ctrl)) return;
  __shared__ int h[256];
  const int nb = 1 << bits;
  const int tid = threadIdx.x;
  const int tile = blockIdx.x, b = blockIdx.y;
  if (tid < nb) h[tid] = 0;
  __syncthreads();
  const int32_t* kb = keys + (size_t)b * N;
  const int base = tile * TILE;
  const uint32_t dmask = (uint32_t)(nb - 1);
  for (int i = tid; i < TILE; i += HT) {
    const int n = base + i;
    if (n < N) atomicAdd(&h[(sort_key(kb[n], K) >> shift) & dmask], 1);
  }
  __syncthreads();
  if (tid < nb) hist[(size_t)b * hstride + (size_t)tid * ntiles + tile] = h[tid];
}

// In-place exclusive scan of one batch row of the digit table (len = bins x
// ntiles entries, digit-major).  One 1024-thread workgroup per batch row;
// each thread owns a contiguous, 4-aligned segment read with 16-byte loads.
__global__ void __launch_bounds__(1024)
sort_scan_kernel(int32_t* __restrict__ hist, int64_t len, int64_t hstride,
                 const int32_t* __restrict__ ctrl) {
  if (loop_done(ctrl)) return;
  __shared__ int wsum[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int32_t* hb = hist + (size_t)blockIdx.x * hstride;
  const int64_t per = ((len + 1023) / 1024 + 3) / 4 * 4;
  const int64_t lo = min((int64_t)tid * per, len);
  const int64_t hi = min(lo + per, len);
  int local = 0;
  int64_t i = lo;
  for (; i + 4 <= hi; i += 4) {
    const int4 v = *reinterpret_cast<const int4*>(hb + i);
    local += v.x + v.y + v.z + v.w;
  }
  for (; i < hi; ++i) local += hb[i];
  int incl = local;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int v = __shfl_up(incl, off, 64);
    if (lane >= off) incl += v;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  if (tid < 64) {
    int v = tid < 16 ? wsum[tid] : 0;
    int inc = v;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      const int u = __shfl_up(inc, off, 64);
      if (tid >= off) inc += u;
    }
    if (tid < 16) wsum[tid] = inc - v;
  }
  __syncthreads();
  int run = wsum[wave] + incl - local;  // exclusive prefix of this thread
  i = lo;
  for (; i + 4 <= hi; i += 4) {
    int4 v = *reinterpret_cast<const int4*>(hb + i);
    int4 o;
    o.x = run; run += v.x;
    o.y = run; run += v.y;
    o.z = run; run += v.z;
    o.w = run; run += v.w;
    *reinterpret_cast<int4*>(hb + i) = o;
  }
  for (; i < hi; ++i) {
    const int v = hb[i];
    hb[i] = run;
    run += v;
  }
}

// Stable rank of every key of one tile by its digit, then a coalesced
// write-out: keys are first placed in LDS in tile-sorted order, then each
// digit's contiguous run is copied to its global slot.
template <int TILE, int ST = Geom<TILE>::ST>
__global__ void __launch_bounds__(ST)
sort_scatter_kernel(const int32_t* __restrict__ keys_in,
                    const int32_t* __restrict__ vals_in,
                    int32_t* __restrict__ keys_out,
                    int32_t* __restrict__ vals_out,
                    const int32_t* __restrict__ offs, int N, int K, int shift,
                    int bits, int ntiles, int64_t hstride,
                    const int32_t* __restrict__ ctrl) {
  constexpr int SW = Geom<TILE>::SW;
  constexpr int PER_WAVE = Geom<TILE>::PER_WAVE;
  constexpr int CHUNKS = Geom<TILE>::CHUNKS;
  if (loop_done(ctrl)) return;
  __shared__ int cnt[SW][256];
  __shared__ int dstart[256];
  __shared__ int gbase[256];
  __shared__ int wtot[4];
  __shared__ int32_t skey[TILE];
  __shared__ int32_t sval[TILE];
  const int nb = 1 << bits;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tile = blockIdx.x, b = blockIdx.y;
  for (int i = tid; i < SW * 256; i += ST) (&cnt[0][0])[i] = 0;
  if (tid < nb) gbase[tid] = offs[(size_t)b * hstride + (size_t)tid * ntiles + tile];
  __syncthreads();

  const int32_t* kb = keys_in + (size_t)b * N;
  const int32_t* vb = vals_in ? vals_in + (size_t)b * N : nullptr;
  const int tbase = tile * TILE;
  const int tn = min(TILE, N - tbase);  // keys in this tile
  const int base = tbase + wave * PER_WAVE;
  int32_t kk[CHUNKS], vv[CHUNKS];
  int rank[CHUNKS], dig[CHUNKS];
  const uint32_t dmask = (uint32_t)(nb - 1);
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int n = base + c * 64 + lane;
    const bool valid = n < N;
    const int32_t key = valid ? kb[n] : 0;
    const int32_t val = valid ? (vb ? vb[n] : n) : 0;
    const uint32_t d = (sort_key(key, K) >> shift) & dmask;
    uint64_t match = __builtin_amdgcn_ballot_w64(valid);
    for (int bit = 0; bit < bits; ++bit) {
      const bool on = (d >> bit) & 1u;
      const uint64_t bal = __builtin_amdgcn_ballot_w64(on);
      match &= on ? bal : ~bal;
    }
    const uint32_t below = lanes_below(match);
    const int old = cnt[wave][d];
    if (valid && below == 0) cnt[wave][d] = old + __popcll(match);
    kk[c] = key;
    vv[c] = val;
    rank[c] = valid ? old + (int)below : -1;
    dig[c] = (int)d;
  }
  __syncthreads();
  // per digit: offsets of each wave inside the digit, and the digit total
  int total = 0;
  if (tid < 256) {
    if (tid < nb) {
      for (int w = 0; w < SW; ++w) {
        const int v = cnt[w][tid];
        cnt[w][tid] = total;
        total += v;
      }
    }
    // exclusive scan of digit totals over the 256 digits (waves 0..3)
    int incl = total;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int u = __shfl_up(incl, off, 64);
      if (lane >= off) incl += u;
    }
    if (lane == 63) wtot[wave] = incl;
    dstart[tid] = incl - total;  // within-wave exclusive prefix for now
  }
  __syncthreads();
  if (tid < 256) {
    int add = 0;
    for (int w = 0; w < wave; ++w) add += wtot[w];
    dstart[tid] += add;
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    if (rank[c] >= 0) {
      const int pos = dstart[dig[c]] + cnt[wave][dig[c]] + rank[c];
      skey[pos] = kk[c];
      sval[pos] = vv[c];
    }
  }
  __syncthreads();
  int32_t* ko = keys_out + (size_t)b * N;
  int32_t* vo = vals_out + (size_t)b * N;
  for (int i = tid; i < tn; i += ST) {
    const int32_t key = skey[i];
    const int d = (int)((sort_key(key, K) >> shift) & dmask);
    const int pos = gbase[d] + (i - dstart[d]);
    ko[pos] = key;
    vo[pos] = sval[i];
  }
}

}  // namespace

SortPlan sort_plan(int64_t B, int64_t N, int64_t K, bool labels_valid) {
  SortPlan p;
  const int64_t span = labels_valid ? K : K + 1;  // K + 1: room for sentinel K
  int bits = 0;
  while ((int64_t(1) << bits) < span) ++bits;
  p.passes = (bits + 7) / 8;
  int shift = 0;
  for (int i = 0; i < p.passes; ++i) {
    const int left = bits - shift;
    const int w = (left + (p.passes - i) - 1) / (p.passes - i);
    p.bits[i] = w;
    p.shift[i] = shift;
    shift += w;
  }
  // 1024-key tiles widen the grid for small N; past 128 tiles per batch row
  // the single-workgroup scan of the (256 x tiles) table costs more than the
  // extra width saves (measured: N = 131072 gains, N = 524288 loses).
  p.tile = N <= 131072 ? 1024 : 4096;
  p.ntiles = (N + p.tile - 1) / p.tile;
  return p;
}

size_t sort_workspace_bytes(int64_t B, int64_t N, int64_t K) {
  const SortPlan p = sort_plan(B, N, K, false);  // the larger of the two plans
  Carve c(nullptr);
  c.take<int32_t>((size_t)B * table_stride(p.ntiles));  // digit table
  const int tmp = p.passes >= 3 ? 2 : (p.passes == 2 ? 1 : 0);
  for (int i = 0; i < tmp; ++i) {
    c.take<int32_t>((size_t)B * N);  // keys
    c.take<int32_t>((size_t)B * N);  // payload
  }
  return c.used;
}

int launch_label_sort(const int32_t* ids, int32_t* sorted_ids, int32_t* perm,
                      int64_t B, int64_t N, int64_t K, bool labels_valid,
                      void* ws, size_t ws_bytes, const int32_t* ctrl,
                      hipStream_t s) {
  if (B == 0 || N == 0) return FKC_OK;
  const size_t need = sort_workspace_bytes(B, N, K);
  if (ws_bytes < need || (need > 0 && ws == nullptr))
    return fail(FKC_ERR_WORKSPACE, "label_sort: workspace %zu < %zu bytes",
                ws_bytes, need);
  if (reinterpret_cast<uintptr_t>(ws) % kWorkspaceAlign != 0)
    return fail(FKC_ERR_WORKSPACE, "label_sort: workspace not %d-byte aligned",
                kWorkspaceAlign);
  const SortPlan p = sort_plan(B, N, K, labels_valid);
  Carve c(ws);
  const int64_t hstride = table_stride(p.ntiles);
  int32_t* hist = c.take<int32_t>((size_t)B * hstride);
  int32_t* tk[2] = {nullptr, nullptr};
  int32_t* tv[2] = {nullptr, nullptr};
  const int tmp = p.passes >= 3 ? 2 : (p.passes == 2 ? 1 : 0);
  for (int i = 0; i < tmp; ++i) {
    tk[i] = c.take<int32_t>((size_t)B * N);
    tv[i] = c.take<int32_t>((size_t)B * N);
  }
  if (p.passes == 0) {  // K == 1 with valid labels: already sorted
    int rc = launch_fill_i32(sorted_ids, 0, B * N, s);
    return rc ? rc : launch_iota_i32(perm, B, N, s);
  }
  const int32_t* kin = ids;
  const int32_t* vin = nullptr;  // identity payload on the first pass
  for (int i = 0; i < p.passes; ++i) {
    const bool last = i == p.passes - 1;
    int32_t* kout = last ? sorted_ids : tk[i % 2];
    int32_t* vout = last ? perm : tv[i % 2];
    const int nb = 1 << p.bits[i];
    dim3 grid((unsigned)p.ntiles, (unsigned)B);
    if (p.tile == 4096)
      hipLaunchKernelGGL(sort_hist_kernel<4096>, grid, dim3(HT), 0, s, kin, hist,
                         (int)N, (int)K, p.shift[i], p.bits[i], (int)p.ntiles,
                         hstride, ctrl);
    else
      hipLaunchKernelGGL(sort_hist_kernel<1024>, grid, dim3(HT), 0, s, kin, hist,
                         (int)N, (int)K, p.shift[i], p.bits[i], (int)p.ntiles,
                         hstride, ctrl);
    int rc = check_launch("sort_hist");
    if (rc) return rc;
    hipLaunchKernelGGL(sort_scan_kernel, dim3((unsigned)B), dim3(1024), 0, s,
                       hist, (int64_t)nb * p.ntiles, hstride, ctrl);
    rc = check_launch("sort_scan");
    if (rc) return rc;
    if (p.tile == 4096)
      hipLaunchKernelGGL(sort_scatter_kernel<4096>, grid, dim3(Geom<4096>::ST), 0,
                         s, kin, vin, kout, vout, hist, (int)N, (int)K,
                         p.shift[i], p.bits[i], (int)p.ntiles, hstride, ctrl);
    else
      hipLaunchKernelGGL(sort_scatter_kernel<1024>, grid, dim3(Geom<1024>::ST), 0,
                         s, kin, vin, kout, vout, hist, (int)N, (int)K,
                         p.shift[i], p.bits[i], (int)p.ntiles, hstride, ctrl);
    rc = check_launch("sort_scatter");
    if (rc) return rc;
    kin = kout;
    vin = vout;
  }
  return FKC_OK;
}

}  // namespace fkc
