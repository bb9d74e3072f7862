// Stable LSD radix sort of cluster labels (replaces torch.sort at
// flash_kmeans_cuda/ops.py:89; the reference asks stable=False, this sort is
// stable so its permutation is reproducible bit for bit).
//
// Keys are labels in [0,K); a label outside that range sorts as K, i.e. after
// every valid label, keeping index order.  The key width is
// bits = ceil(log2(K+1)) so the sentinel has a bin, or ceil(log2(K)) when the
// caller vouches that every label is valid (labels straight from the assign
// kernel), split into passes of at most 8 bits.
//
// Each pass is a single kernel that places its tile's keys using a chained
// scan with decoupled look-back (Merrill & Garland, "Single-pass Parallel
// Prefix Scan with Decoupled Look-back", 2016; the radix-sort form is Adinets
// & Merrill, "Onesweep", 2022).  A pass needs the row's global digit counts
// before it places anything:
//   fused first pass (every tile of the launch resident at once, at most 256
//                   tiles): each tile adds its digit counts of every pass to
//                   the row's global counts, then arrives at a row barrier;
//                   it waits there only after its own look-back, when the
//                   other tiles have long arrived.
//   sort_upsweep  : (larger grids) one read of the keys counts the digits of
//                   every pass into the global counts before the passes.
//   sort_onesweep : ranks its tile's keys stably by digit (per 64-key chunk,
//                   every lane ORs its lane bit into the wave's LDS word for
//                   its digit and reads the word back: the mask of lanes
//                   holding its digit, "multi-split"), publishes its
//                   per-digit counts, then walks back over earlier tiles'
//                   status words, adding their counts until it meets an
//                   inclusive prefix, and publishes its own inclusive prefix.
//                   Keys are placed in LDS in tile-sorted order and each
//                   digit's run is copied to its global slot, so writes are
//                   runs of consecutive addresses.  A resident grid takes the
//                   block index as the tile's place in the chain; a larger
//                   one takes the next index from a counter, so every tile a
//                   walk waits for is already running.
// A status word is 64 bits: flag in bits 63..62 (published count, or
// inclusive prefix), the call's epoch in bits 61..32, count in bits 31..0,
// read and written with relaxed agent-scope atomics, so a reader sees flag,
// epoch and count together and no fence is needed.  A word of an earlier
// call carries another epoch and reads as unpublished, so status words are
// never cleared between calls; the tile counters and the barrier's arrival
// counter only grow, and a call offsets them by its sequence number.
// Every wait is bounded.  A digit whose walk runs past the spin limit stops
// waiting, and the workgroup counts that digit's keys in every earlier tile
// straight from the pass's input (written by the previous launch, so always
// complete); a tile whose barrier wait runs out counts the whole row's
// digits itself.  Either gives the same numbers as the wait, so the output
// is correct either way and every workgroup exits; the workspace's first
// word counts how often a recount ran (zero in a normal run).
//
// The global digit counts accumulate into one of two buffers (the parity of
// the call's sequence number); each call clears the other one, which the
// previous call used and the next one will.  A standalone call clears the
// whole control region first.
// The carried payload is the original index; the last pass writes the
// user's sorted_ids / perm.
#include "device_util.hpp"
#include "fkc_internal.hpp"

#include <algorithm>
#include <atomic>

namespace fkc {
namespace {

constexpr int MAXP = 4;           // passes at most (31-bit keys, 8-bit digits)
constexpr int UPT = 512;          // threads of the upsweep kernel
constexpr uint64_t ST_AGG = 1ull << 62;  // the tile's own digit count
constexpr uint64_t ST_INC = 2ull << 62;  // inclusive prefix over tiles 0..t
constexpr uint64_t ST_CNT = 0xffffffffull;  // count field
constexpr int64_t EPOCHS = (1ll << 30) - 1;  // epochs 1 .. EPOCHS; 0 = cleared
constexpr int SPIN_LIMIT = 1 << 18;  // empty polls per wait (< 1 s)
#ifndef FKC_SORT_LB
#define FKC_SORT_LB 4
#endif
constexpr int LB = FKC_SORT_LB;      // status words read per look-back step
// Grids of at most this many tiles (per launch), and at most the device
// holds at once (sort_resident_tiles), are resident at once, so a tile may
// take its block index as its place in the chain and the first pass may
// wait at a row barrier.
constexpr int64_t STATIC_TILES_MAX = 256;
// Per-row counters (uint64): the tile counter of each pass, then the
// arrival counter of the fused first pass.
constexpr int CTR = 8;
constexpr int CTR_ARRIVE = MAXP;

struct PassDesc {
  int passes;
  int bits[MAXP];
  int shift[MAXP];
};

// Threads of the onesweep kernel per tile size.
template <int TILE_>
struct Geom {
  static constexpr int TILE = TILE_;
  static constexpr int ST = TILE_ >= 8192 ? 1024 : (TILE_ >= 4096 ? 512 : 256);
  static constexpr int SW = ST / 64;
  static constexpr int PER_WAVE = TILE / SW;
  static constexpr int CHUNKS = PER_WAVE / 64;
  static_assert(CHUNKS >= 1 && PER_WAVE % 64 == 0, "onesweep geometry");
};

__device__ inline uint32_t sort_key(int32_t id, int K) {
  return (uint32_t)id < (uint32_t)K ? (uint32_t)id : (uint32_t)K;
}

// Workspace layout, shared by the size query and the launcher.  err, gcnt,
// ctr and status are consecutive: the control region a reset clears.
struct SortBufs {
  int32_t* err;      // [1] recounts after a wait ran out of spins
  int32_t* gcnt;     // [2 phases][B][MAXP][256] global digit counts
  uint64_t* ctr;     // [B][CTR] tile counters, arrival counter
  uint64_t* status;  // [B][P][ntiles][256] tile status words
  int32_t* tk[2];    // ping buffers: keys
  int32_t* tv[2];    //               payload
  int64_t gphase;    // int32 entries per phase of gcnt
  int64_t slen;      // status words per batch row
  int64_t nctl;      // int32 words of the control region
};

SortBufs carve_sort(void* ws, int64_t B, int64_t N, int64_t K, size_t* used) {
  const SortPlan p = sort_plan(B, N, K, false);  // the larger of the two plans
  Carve c(ws);
  SortBufs s{};
  s.gphase = B * MAXP * 256;
  s.err = c.take<int32_t>((size_t)64 + 2 * s.gphase);
  s.gcnt = s.err ? s.err + 64 : nullptr;
  s.ctr = c.take<uint64_t>((size_t)B * CTR);
  s.slen = (int64_t)p.passes * p.ntiles * 256;
  s.status = c.take<uint64_t>((size_t)B * s.slen);
  s.nctl = (int64_t)(c.used / sizeof(int32_t));
  const int tmp = p.passes >= 3 ? 2 : (p.passes == 2 ? 1 : 0);
  for (int i = 0; i < tmp; ++i) {
    s.tk[i] = c.take<int32_t>((size_t)B * N);
    s.tv[i] = c.take<int32_t>((size_t)B * N);
  }
  if (used) *used = c.used;
  return s;
}

// Digit counts of every pass over this workgroup's keys, added into
// gcnt_cur; workgroup 0 of a row also clears the row's other-phase counts.
__global__ void __launch_bounds__(UPT)
sort_upsweep_kernel(const int32_t* __restrict__ keys, int N, int K,
                    PassDesc pd, int per_wg, int32_t* __restrict__ gcnt_cur,
                    int32_t* __restrict__ gcnt_next,
                    const int32_t* __restrict__ ctrl) {
  if (loop_done(ctrl)) return;
  __shared__ int h[MAXP][256];
  const int tid = threadIdx.x;
  const int w = blockIdx.x, b = blockIdx.y;
  for (int i = tid; i < MAXP * 256; i += UPT) (&h[0][0])[i] = 0;
  if (w == 0)
    for (int i = tid; i < MAXP * 256; i += UPT)
      gcnt_next[(size_t)b * MAXP * 256 + i] = 0;
  __syncthreads();
  const int32_t* kb = keys + (size_t)b * N;
  const int lo = w * per_wg, hi = min(lo + per_wg, N);
  for (int n = lo + tid; n < hi; n += UPT) {
    const uint32_t key = sort_key(kb[n], K);
    for (int p = 0; p < pd.passes; ++p)
      atomicAdd(&h[p][(key >> pd.shift[p]) & ((1u << pd.bits[p]) - 1u)], 1);
  }
  __syncthreads();
  for (int i = tid; i < pd.passes * 256; i += UPT) {
    const int v = (&h[0][0])[i];
    if (v) atomicAdd(&gcnt_cur[(size_t)b * MAXP * 256 + i], v);
  }
}

// Exclusive scan over the 256 digits of two values at once (digit = tid for
// threads 0..255; wtot holds 2 x 4 wave totals).  Every thread of the
// workgroup calls it (it contains a barrier); waves past the fourth pass
// zeros and their results are unused.  Returns the exclusive prefixes.
// drain: every thread first waits for its outstanding global memory
// operations, so that they are complete once the barrier is passed.
__device__ inline int2 scan256x2(int a, int c, int* wtot, int tid,
                                 bool drain = false) {
  const int lane = tid & 63, wave = tid >> 6;
  const int ia = wave_incl_scan(a), ic = wave_incl_scan(c);
  if (lane == 63 && wave < 4) {
    wtot[wave] = ia;
    wtot[4 + wave] = ic;
  }
  if (drain) drain_before_announce();
  __syncthreads();
  int ba = 0, bc = 0;
  for (int w = 0; w < min(wave, 4); ++w) {
    ba += wtot[w];
    bc += wtot[4 + w];
  }
  return int2{ba + ia - a, bc + ic - c};
}

struct SweepArgs {
  const int32_t* keys_in;
  const int32_t* vals_in;  // null: the identity payload (first pass)
  int32_t* keys_out;
  int32_t* vals_out;
  int32_t* gcnt;           // this call's digit counts, row stride MAXP*256
  int32_t* gnext;          // the other phase (cleared by a fused pass)
  uint64_t* status;        // this pass's status words, row stride slen
  int64_t slen;
  uint64_t* ctr;           // per-row counters, row stride CTR
  int32_t* err;
  const int32_t* ctrl;
  PassDesc pd;
  int64_t seq;             // sort calls on this workspace since its reset
  uint64_t tag;            // this call's epoch, in place (bits 61..32)
  int N, K, pass, spin_limit;
  int dyn_tiles;           // tile index from the row's counter
  int fuse;                // first pass that also counts every pass's digits
};

// Sum of v over the q lanes of the calling lane's group (q in {1, 2, 4, 8};
// groups are aligned runs of q lanes), returned to every lane of the group:
// DPP adds over quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror.
__device__ inline int group_sum(int v, int q) {
  if (q >= 2) v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
  if (q >= 4) v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
  if (q >= 8) v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
  return v;
}

// Published for this call: flag set and this call's epoch.
__device__ inline bool st_published(uint64_t v, uint64_t tag) {
  const uint64_t hi = v & ~ST_CNT;
  return hi == (ST_AGG | tag) || hi == (ST_INC | tag);
}

template <int TILE, int ST = Geom<TILE>::ST>
__global__ void __launch_bounds__(ST) sort_onesweep_kernel(SweepArgs a) {
  constexpr int SW = Geom<TILE>::SW;
  constexpr int PER_WAVE = Geom<TILE>::PER_WAVE;
  constexpr int CHUNKS = Geom<TILE>::CHUNKS;
  __shared__ int cnt[SW][256];
  __shared__ unsigned long long lmask[SW][256];  // ranking: lanes per digit
  __shared__ int hx[MAXP - 1][256];  // fused: digit counts of later passes
  __shared__ int gbase[256];
  __shared__ int dstart[256];
  __shared__ int wtot[8];
  __shared__ int s_tot[256];   // the tile's count per digit
  __shared__ int s_excl[256];  // exclusive prefix over earlier tiles; -1: stopped
  __shared__ int s_tile;
  __shared__ int s_recount;  // a digit of this tile stopped waiting
  __shared__ int s_short;    // the row barrier's wait ran out (fused)
  __shared__ int32_t skey[TILE];
  __shared__ int32_t sval[TILE];
  const int N = a.N, K = a.K;
  // Pass parameters are grid-uniform: scalar registers (read from the
  // argument block once, not per chunk).
  const int npass = __builtin_amdgcn_readfirstlane(a.pd.passes);
  const int shift = __builtin_amdgcn_readfirstlane(a.pd.shift[a.pass]);
  const int bits = __builtin_amdgcn_readfirstlane(a.pd.bits[a.pass]);
  const bool fuse = a.fuse != 0;
  const int nb = 1 << bits;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = blockIdx.y;
  const int64_t ntiles = gridDim.x;
  int32_t* grow = a.gcnt + (size_t)b * MAXP * 256;
  uint64_t* crow = a.ctr + (size_t)b * CTR;
  uint64_t* srow = a.status + (size_t)b * a.slen;
  const int32_t* kb = a.keys_in + (size_t)b * N;
  const int32_t* vb = a.vals_in ? a.vals_in + (size_t)b * N : nullptr;
  // Loads are unconditional (index clamped to the row, a first pass
  // re-reading the keys where it has no payload) so that all of them are in
  // flight at once: a load under a branch makes the compiler wait for it at
  // the join.  Lanes past N are masked in the ranking; the identity payload
  // is substituted at placement.
  const int32_t* vsrc = vb ? vb : kb;
  int32_t kk[CHUNKS], vv[CHUNKS];
  auto load_tile = [&](int t) {
    const int base = t * TILE + wave * PER_WAVE;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int n = min(base + c * 64 + lane, N - 1);
      kk[c] = kb[n];
      vv[c] = vsrc[n];
    }
  };
  // A resident grid's tile is its block index: its keys are in flight
  // before the control word is even read (a finished loop then drops them).
  if (!a.dyn_tiles) load_tile((int)blockIdx.x);
  if (loop_done(a.ctrl)) return;
  // The pass's global digit count does not depend on the tile: its load is
  // in flight together with the tile-counter atomic.  (A fused pass has it
  // only after the row barrier.)
  int gc = (!fuse && tid < nb) ? grow[a.pass * 256 + tid] : 0;
  for (int i = tid; i < SW * 256; i += ST) {
    (&cnt[0][0])[i] = 0;
    (&lmask[0][0])[i] = 0ull;
  }
  if (fuse)
    for (int i = tid; i < (MAXP - 1) * 256; i += ST) (&hx[0][0])[i] = 0;
  // Tile index: with dyn_tiles, the order in which workgroups start (the
  // counter grows by ntiles per call), so every tile a walk waits for is
  // already running; when the whole grid is resident at once, the block
  // index (one round trip less).
  if (tid == 0) {
    s_tile = a.dyn_tiles
                 ? (int)(atomicAdd(reinterpret_cast<unsigned long long*>(
                                       crow + a.pass),
                                   1ull) -
                         (unsigned long long)a.seq * ntiles)
                 : (int)blockIdx.x;
    s_recount = 0;
    s_short = 0;
  }
  __syncthreads();
  const int tile = s_tile;
  // A counter out of step with seq (a caller that broke the sequence
  // contract) must not send the workgroup outside the row: it leaves, and
  // the workspace's second word records it.
  if (tile < 0 || tile >= ntiles) {
    if (tid == 0) atomicAdd(a.err + 1, 1);
    return;
  }
  if (a.dyn_tiles) load_tile(tile);

  const int tbase = tile * TILE;
  const int tn = min(TILE, N - tbase);  // keys in this tile
  const int base = tbase + wave * PER_WAVE;
  int rank[CHUNKS], dig[CHUNKS];
  uint64_t match[CHUNKS];
  int lead[CHUNKS];
  const uint32_t dmask = (uint32_t)(nb - 1);
  // Later passes' digit fields (fused first pass).
  uint32_t hsh[MAXP - 1], hmask[MAXP - 1];
#pragma unroll
  for (int p = 0; p < MAXP - 1; ++p) {
    hsh[p] = (uint32_t)__builtin_amdgcn_readfirstlane(a.pd.shift[p + 1]);
    hmask[p] =
        (1u << __builtin_amdgcn_readfirstlane(a.pd.bits[p + 1])) - 1u;
  }
  // Per 64-key chunk: the mask of lanes holding the lane's digit
  // ("multi-split"): every lane ORs its lane bit into the wave's LDS word
  // for its digit and reads the word back, and the word is cleared for the
  // next chunk (an OR does not depend on the order of the lanes, and a
  // wave's LDS operations execute in issue order, so the read sees exactly
  // this chunk's bits; one LDS round trip instead of a ballot per digit
  // bit, about 11 vector instructions each).  The digit's first lane then
  // adds the group's size to the wave's count with an LDS atomic that
  // returns the count before it; the atomics of all chunks issue back to
  // back and each returns the count after the wave's earlier chunks.
  const unsigned long long mybit = 1ull << lane;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const bool valid = base + c * 64 + lane < N;
    const uint32_t d = (sort_key(kk[c], K) >> shift) & dmask;
    unsigned long long* w = &lmask[wave][d];
    __hip_atomic_fetch_or(w, valid ? mybit : 0ull, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_WORKGROUP);
    match[c] = __hip_atomic_load(w, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_WORKGROUP);
    __hip_atomic_store(w, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    dig[c] = (int)d;
  }
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const bool valid = base + c * 64 + lane < N;
    const uint32_t key = sort_key(kk[c], K);
    const uint32_t d = (uint32_t)dig[c];
    const uint64_t m = match[c];
    int o = 0;
    if (valid && lanes_below(m) == 0) o = atomicAdd(&cnt[wave][d], __popcll(m));
    lead[c] = o;
    if (fuse && valid) {
#pragma unroll
      for (int p = 0; p < MAXP - 1; ++p)
        if (p + 1 < npass) atomicAdd(&hx[p][(key >> hsh[p]) & hmask[p]], 1);
    }
  }
  // The count before the chunk reaches the digit's other lanes from its
  // first lane.
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const uint64_t m = match[c];
    lead[c] = __shfl(lead[c], m ? (int)__builtin_ctzll(m) : lane, 64);
  }
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const bool valid = base + c * 64 + lane < N;
    rank[c] = (lead[c] + (int)lanes_below(match[c])) | (valid ? 0 : -1);
  }
  __syncthreads();

  // Per digit: the waves' offsets inside the digit and the tile's count,
  // published at once so later tiles can move on.  A fused pass also adds
  // the tile's counts of every pass into the row's global counts and makes
  // them visible before the workgroup arrives at the row barrier.
  int total = 0;
  if (tid < 256) {
    if (tid < nb) {
      int v[SW];
#pragma unroll
      for (int w = 0; w < SW; ++w) v[w] = cnt[w][tid];
#pragma unroll
      for (int w = 0; w < SW; ++w) {
        cnt[w][tid] = total;
        total += v[w];
      }
      __hip_atomic_store(srow + (size_t)tile * 256 + tid,
                         (tile == 0 ? ST_INC : ST_AGG) | a.tag | (uint64_t)total,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (fuse && total) atomicAdd(grow + tid, total);
      s_tot[tid] = total;
    }
    if (fuse) {
      for (int p = 1; p < a.pd.passes; ++p) {
        const int v = hx[p - 1][tid];
        if (v) atomicAdd(grow + p * 256 + tid, v);
      }
    }
  }
  // The first tile of a fused row clears the other phase's counts (used by
  // the previous call, which has finished, and next by the following call).
  if (fuse && tile == 0)
    for (int i = tid; i < MAXP * 256; i += ST)
      a.gnext[(size_t)b * MAXP * 256 + i] = 0;
  // Tile-local and global exclusive digit prefixes.  A fused pass's adds
  // are agent-scope atomics, performed where every workgroup reads them;
  // waiting for their completion (drain) before the scan's barrier orders
  // them before the arrival below (a release fence would also write back
  // this XCD's L2, which cost ~0.1 us per wave).
  const int2 pre = scan256x2(total, gc, wtot, tid, fuse);
  if (fuse && tid == 0)
    __hip_atomic_fetch_add(crow + CTR_ARRIVE, 1ull, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  // Look-back over earlier tiles' status words, per digit.  With one lane
  // per digit the lane reads LB predecessors at once (one round trip per
  // window), then takes them newest first: counts add up until an
  // inclusive prefix (or tile 0); a word not yet published ends the window,
  // and the walk polls again from it.  With more threads than digits, q
  // lanes per digit (at most 8) walk together: lane j of a digit's group
  // reads tiles t - j*LB .. t - j*LB - LB + 1, so one round trip covers
  // q*LB predecessors, and every lane of the group derives the same walk
  // state from a ballot and DPP sums.
  int q = 1;
  while (q < 8 && nb * q * 2 <= ST) q <<= 1;
  bool stopped = false;  // this digit's walk ran out of spins (tid < nb)
  if (q == 1) {
    if (tid < nb) {
      int64_t excl = 0;
      if (tile > 0) {
        const uint64_t* col = srow + tid;
        int spins = 0;  // one budget for the whole walk
        int t = tile - 1;
        for (;;) {
          if (spins >= a.spin_limit) {
            stopped = true;
            break;
          }
          uint64_t v[LB];
#pragma unroll
          for (int i = 0; i < LB; ++i)
            v[i] = t - i >= 0 ? __hip_atomic_load(col + (size_t)(t - i) * 256,
                                                  __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT)
                              : 0ull;
          int used = 0;       // words of the window consumed
          bool done = false;  // an inclusive prefix (or tile 0) was reached
#pragma unroll
          for (int i = 0; i < LB; ++i) {
            if (!st_published(v[i], a.tag)) break;
            excl += (int64_t)(v[i] & ST_CNT);
            used = i + 1;
            if ((v[i] & ST_INC) || t - i == 0) {
              done = true;
              break;
            }
          }
          if (done) break;
          t -= used;
          if (used < LB) {  // the next word is not published yet
            ++spins;
            __builtin_amdgcn_s_sleep(1);
          }
        }
        if (stopped)
          s_recount = 1;
        else
          __hip_atomic_store(srow + (size_t)tile * 256 + tid,
                             ST_INC | a.tag | (uint64_t)(excl + total),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      dstart[tid] = pre.x;
      gbase[tid] = pre.y + (int)excl - pre.x;  // fused: pre.y == 0 here
    }
  } else {
    const int ld = tid / q, lj = tid % q;  // digit, lane in its group
    const int g0 = lane - lj;              // the group's first lane (q | 64)
    bool gstop = false;                    // the group's walk ran out of spins
    int64_t gexcl = 0;
    const uint64_t* col = srow + (ld < nb ? ld : 0);
    int spins = 0;  // one budget for the whole walk
    int t = tile - 1;
    bool gdone = !(ld < nb && tile > 0);
    while (__builtin_amdgcn_ballot_w64(!gdone) != 0) {  // wave-uniform
      if (!gdone && spins >= a.spin_limit) {
        gstop = true;
        gdone = true;
      }
      const int tb = t - lj * LB;  // newest tile of this lane's share
      uint64_t v[LB];
#pragma unroll
      for (int i = 0; i < LB; ++i)
        v[i] = !gdone && tb - i >= 0
                   ? __hip_atomic_load(col + (size_t)(tb - i) * 256,
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                   : 0ull;
      uint32_t sum = 0;  // counts of this lane's consumed words (< 2^32)
      int used = 0;      // words of the share consumed
      bool inc = false;  // an inclusive prefix (or tile 0) was reached
      bool go = true;
#pragma unroll
      for (int i = 0; i < LB; ++i) {
        if (go) {
          if (!st_published(v[i], a.tag)) {
            go = false;
          } else {
            sum += (uint32_t)(v[i] & ST_CNT);
            used = i + 1;
            if ((v[i] & ST_INC) || tb - i == 0) {
              inc = true;
              go = false;
            }
          }
        }
      }
      // The group's first lane js whose share did not pass through whole:
      // lanes 0 .. js consumed their words this step (lanes before js all
      // LB of them), so the step's counts, words consumed and inclusive
      // flag are group sums over those lanes.
      const bool full = !gdone && used == LB && !inc;
      const uint64_t nf = __builtin_amdgcn_ballot_w64(!full);
      const uint32_t mg = (uint32_t)(nf >> g0) & ((1u << q) - 1u);
      const int js = mg ? __builtin_ctz(mg) : q;
      const bool mine = lj <= js;
      const uint32_t tot = (uint32_t)group_sum(mine ? (int)sum : 0, q);
      const int pk = group_sum(mine ? used | (inc ? 256 : 0) : 0, q);
      if (!gdone) {
        gexcl += tot;
        if (pk >> 8) {
          gdone = true;
        } else {
          t -= pk & 255;
          if (js < q) {  // a word not yet published
            ++spins;
            __builtin_amdgcn_s_sleep(1);
          }
        }
      }
    }
    if (lj == 0 && ld < nb) {
      if (tile > 0) {
        if (gstop)
          s_recount = 1;
        else
          __hip_atomic_store(srow + (size_t)tile * 256 + ld,
                             ST_INC | a.tag | (uint64_t)(gexcl + s_tot[ld]),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      s_excl[ld] = gstop ? -1 : (int)gexcl;
    }
    __syncthreads();
    if (tid < nb) {
      const int e = s_excl[tid];
      stopped = e < 0;
      dstart[tid] = pre.x;
      gbase[tid] = pre.y + (stopped ? 0 : e) - pre.x;  // fused: pre.y == 0
    }
  }
  __syncthreads();
  if (s_recount) {  // workgroup-uniform; never taken in a normal run
    // Count the digits of keys 0 .. tbase-1 of this pass's input (the
    // earlier tiles) in LDS; a stopped digit's exclusive prefix is its
    // count.  skey is free until the placement below.
    int* rc = skey;
    for (int i = tid; i < 256; i += ST) rc[i] = 0;
    __syncthreads();
    for (int n = tid; n < tbase; n += ST)
      atomicAdd(&rc[(sort_key(kb[n], K) >> shift) & dmask], 1);
    __syncthreads();
    if (stopped) {
      const int excl = rc[tid];
      __hip_atomic_store(srow + (size_t)tile * 256 + tid,
                         ST_INC | a.tag | (uint64_t)(excl + total),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      gbase[tid] = pre.y + excl - pre.x;
    }
    if (tid == 0) atomicAdd(a.err, 1);
    __syncthreads();
  }
  if (fuse) {  // workgroup-uniform
    // Row barrier: every tile of the row has added its counts once the
    // arrival counter reaches ntiles more than before this call.
    if (tid == 0) {
      const uint64_t want = (uint64_t)(a.seq + 1) * (uint64_t)ntiles;
      int spins = 0;
      int ok = 0;
      while (spins < a.spin_limit) {
        if (__hip_atomic_load(crow + CTR_ARRIVE, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT) >= want) {
          ok = 1;
          break;
        }
        ++spins;
        __builtin_amdgcn_s_sleep(1);
      }
      s_short = !ok;
    }
    __syncthreads();
    if (!s_short) {
      // Agent-scope atomic loads read the counts where the adds were
      // performed (no stale cached copy).
      gc = tid < nb ? __hip_atomic_load(grow + tid, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT)
                    : 0;
    } else {
      // Count the whole row's digits of this pass from its input.
      int* rc = skey;
      for (int i = tid; i < 256; i += ST) rc[i] = 0;
      __syncthreads();
      for (int n = tid; n < N; n += ST)
        atomicAdd(&rc[(sort_key(kb[n], K) >> shift) & dmask], 1);
      __syncthreads();
      gc = tid < nb ? rc[tid] : 0;
      if (tid == 0) atomicAdd(a.err, 1);
      __syncthreads();
    }
    const int2 g = scan256x2(gc, 0, wtot, tid);
    if (tid < nb) gbase[tid] += g.x;
  }
  // Placement in tile order, without branches so that every chunk's LDS
  // reads are in flight at once: a key past N (only in a short last tile)
  // goes to slot TILE - 1, which is at or past tn and never read.
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int d = dig[c];
    const int pos =
        rank[c] >= 0 ? dstart[d] + cnt[wave][d] + rank[c] : TILE - 1;
    skey[pos] = kk[c];
    sval[pos] = vb ? vv[c] : base + c * 64 + lane;
  }
  __syncthreads();
  int32_t* ko = a.keys_out + (size_t)b * N;
  int32_t* vo = a.vals_out + (size_t)b * N;
  // Copy out: every slot is read (in LDS bounds; a slot past tn yields some
  // digit in range) and only the stores are masked.
  constexpr int PER_T = TILE / ST;
  int32_t ok[PER_T], ov[PER_T], op[PER_T];
#pragma unroll
  for (int j = 0; j < PER_T; ++j) {
    ok[j] = skey[tid + j * ST];
    ov[j] = sval[tid + j * ST];
  }
#pragma unroll
  for (int j = 0; j < PER_T; ++j)
    op[j] = gbase[(sort_key(ok[j], K) >> shift) & dmask] + tid + j * ST;
#pragma unroll
  for (int j = 0; j < PER_T; ++j) {
    if (tid + j * ST < tn) {
      ko[op[j]] = ok[j];
      vo[op[j]] = ov[j];
    }
  }
}

template <int TILE>
void launch_onesweep(dim3 grid, hipStream_t s, const SweepArgs& a) {
  hipLaunchKernelGGL((sort_onesweep_kernel<TILE>), grid, dim3(Geom<TILE>::ST),
                     0, s, a);
}

// Onesweep workgroups of this tile size one CU holds at once (the occupancy
// API), read once per device; 1 without a device.
template <int TILE>
int onesweep_per_cu() {
  constexpr int kMaxDev = 64;
  static std::atomic<int> cache[kMaxDev];  // 0: not read yet
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) {
    (void)hipGetLastError();
    return 1;
  }
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, reinterpret_cast<const void*>(&sort_onesweep_kernel<TILE>),
            Geom<TILE>::ST, 0) != hipSuccess ||
        n < 1)
      n = 1;
    (void)hipGetLastError();
    cache[dev].store(n, std::memory_order_relaxed);
    v = n;
  }
  return v;
}

}  // namespace

// Tiles of one launch that run at once on the current device: its CUs times
// the onesweep workgroups per CU, capped at STATIC_TILES_MAX.  A grid within
// it may take block indices as chain positions and wait at a row barrier
// (every tile it waits for is running); a larger one takes positions from a
// counter and counts its digits in an upsweep.  A device shared with other
// work can still hold fewer: the waits are bounded, so that costs time, not
// correctness (the recount word reports it).
int64_t sort_resident_tiles(int tile) {
  int per_cu = 1;
  switch (tile) {
    case 256: per_cu = onesweep_per_cu<256>(); break;
    case 512: per_cu = onesweep_per_cu<512>(); break;
    case 1024: per_cu = onesweep_per_cu<1024>(); break;
    case 2048: per_cu = onesweep_per_cu<2048>(); break;
    case 8192: per_cu = onesweep_per_cu<8192>(); break;
    default: per_cu = onesweep_per_cu<4096>(); break;
  }
  return std::min<int64_t>(STATIC_TILES_MAX,
                           (int64_t)device_shape().cus * per_cu);
}

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
  // 4096-key tiles: a pass costs a few dependent memory round trips per
  // tile plus about 20 ns of look-back chain per tile, so fewer, larger
  // tiles win even when they leave CUs idle (measured at N = 524288,
  // K = 8192: 52 / 32 / 21 / 16 / 13.5 us per pass for 256 .. 4096-key
  // tiles).  8192-key tiles lose: with 16 keys per thread a pass took
  // 16.4 us, and on 1024 threads (8 keys each) the 89 KB workgroup runs
  // alone on its CU (the whole c5 sort 37.3 vs 35.1 us).  With at most
  // 65536 keys in all the chain is short and smaller tiles shorten each
  // tile's own work (1024 / 2048 / 4096-key tiles, us per pass: 8.6 / 10.4
  // / 10.7 at B x N = 32768; 8.6 / 9.5 / 9.4 at 65536; but 10.2 / 10.2 /
  // 9.8 at 131072 and 12.0 / 10.4 / 9.6 at 8 x 65536), and up to 32768
  // keys 512-key tiles shorten it once more (Lloyd loop, us per iteration
  // with 512 / 1024-key tiles: 30.8-31.1 / 31.9-32.6 at 4096 keys, 30.0-30.2
  // / 30.3-30.7 at 32768; at 65536 they lose 2.5 us).  With the ranking by
  // LDS lane masks a tile's own work is cheaper, and the balance moved:
  // 1024-key tiles at 32768 keys (27.5-28.2 against 28.3-28.8 us; 256-key
  // tiles at 4096 keys were within noise).  Batches of short
  // rows take 2048-key tiles when a row needs at most 32 of them and the
  // grid stays resident: the chain stays short and each tile's own work
  // halves (8 x 65536 keys: 118.8-119.3 against 120.2-120.3 us per
  // iteration; with longer chains 2048 loses: 1 x 131072 +1 us, 1 x 524288
  // +5 us).  FKC_SORT_TILE overrides.
  const int64_t t2k = (N + 2047) / 2048;
  int tile = B * N <= 16384   ? 512
             : B * N <= 65536 ? 1024
             : (B > 1 && t2k <= 32 && B * t2k <= sort_resident_tiles(2048))
                 ? 2048
                              : 4096;
  if (const int o = sort_tile_override()) tile = o;
  p.tile = tile;
  p.ntiles = (N + p.tile - 1) / p.tile;
  return p;
}

size_t sort_workspace_bytes(int64_t B, int64_t N, int64_t K) {
  size_t used = 0;
  carve_sort(nullptr, B, N, K, &used);
  return used;
}

int launch_label_sort(const int32_t* ids, int32_t* sorted_ids, int32_t* perm,
                      int64_t B, int64_t N, int64_t K, bool labels_valid,
                      void* ws, size_t ws_bytes, const int32_t* ctrl,
                      hipStream_t s, int64_t seq) {
  if (B == 0 || N == 0) return FKC_OK;
  const size_t need = sort_workspace_bytes(B, N, K);
  if (ws_bytes < need || (need > 0 && ws == nullptr))
    return fail(FKC_ERR_WORKSPACE, "label_sort: workspace %zu < %zu bytes",
                ws_bytes, need);
  if (reinterpret_cast<uintptr_t>(ws) % kWorkspaceAlign != 0)
    return fail(FKC_ERR_WORKSPACE, "label_sort: workspace not %d-byte aligned",
                kWorkspaceAlign);
  const SortPlan p = sort_plan(B, N, K, labels_valid);
  if (p.passes == 0) {  // K == 1 with valid labels: already sorted
    int rc = launch_fill_i32(sorted_ids, 0, B * N, s);
    return rc ? rc : launch_iota_i32(perm, B, N, s);
  }
  SortBufs w = carve_sort(ws, B, N, K, nullptr);
  if (seq < 0) {
    int rc = launch_fill_i32(w.err, 0, w.nctl, s);
    if (rc) return rc;
    seq = 0;
  }
  int32_t* gcur = w.gcnt + (size_t)(seq & 1) * w.gphase;
  int32_t* gnext = w.gcnt + (size_t)((seq & 1) ^ 1) * w.gphase;
  PassDesc pd{};
  pd.passes = p.passes;
  for (int i = 0; i < p.passes; ++i) {
    pd.bits[i] = p.bits[i];
    pd.shift[i] = p.shift[i];
  }
  // A grid that is resident at once takes block indices as tiles and counts
  // the digits in its first pass; a larger one needs the upsweep.
  const bool resident = B * p.ntiles <= sort_resident_tiles(p.tile);
  const bool fuse = resident && sort_fuse_override();
  int rc = FKC_OK;
  if (!fuse) {
    // Upsweep: about 128 workgroups per batch row, 1024..8192 keys each.
    int per_wg = 1024;
    while (per_wg < 8192 && (N + per_wg - 1) / per_wg > 128) per_wg <<= 1;
    dim3 ugrid((unsigned)((N + per_wg - 1) / per_wg), (unsigned)B);
    hipLaunchKernelGGL(sort_upsweep_kernel, ugrid, dim3(UPT), 0, s, ids,
                       (int)N, (int)K, pd, per_wg, gcur, gnext, ctrl);
    rc = check_launch("sort_upsweep");
    if (rc) return rc;
  }

  SweepArgs a{};
  a.gcnt = gcur;
  a.gnext = gnext;
  a.slen = w.slen;
  a.ctr = w.ctr;
  a.err = w.err;
  a.ctrl = ctrl;
  a.pd = pd;
  a.seq = seq;
  a.tag = (uint64_t)(1 + seq % EPOCHS) << 32;
  a.N = (int)N;
  a.K = (int)K;
  // FKC_SORT_SPIN (tests): a smaller spin budget; 0 sends every wait to its
  // recount.
  a.spin_limit = sort_spin_override(SPIN_LIMIT);
  a.dyn_tiles = resident ? 0 : 1;
  a.keys_in = ids;
  a.vals_in = nullptr;  // identity payload on the first pass
  for (int i = 0; i < p.passes; ++i) {
    const bool last = i == p.passes - 1;
    a.keys_out = last ? sorted_ids : w.tk[i % 2];
    a.vals_out = last ? perm : w.tv[i % 2];
    a.status = w.status + (size_t)i * p.ntiles * 256;
    a.pass = i;
    a.fuse = fuse && i == 0 ? 1 : 0;
    dim3 grid((unsigned)p.ntiles, (unsigned)B);
    switch (p.tile) {
      case 256: launch_onesweep<256>(grid, s, a); break;
      case 512: launch_onesweep<512>(grid, s, a); break;
      case 1024: launch_onesweep<1024>(grid, s, a); break;
      case 2048: launch_onesweep<2048>(grid, s, a); break;
      case 8192: launch_onesweep<8192>(grid, s, a); break;
      default: launch_onesweep<4096>(grid, s, a); break;
    }
    rc = check_launch("sort_onesweep");
    if (rc) return rc;
    a.keys_in = a.keys_out;
    a.vals_in = a.vals_out;
  }
  return FKC_OK;
}

int label_sort_reset(void* ws, int64_t B, int64_t N, int64_t K,
                     hipStream_t s) {
  int32_t* p = nullptr;
  int64_t n = 0;
  label_sort_reset_region(ws, B, N, K, &p, &n);
  return launch_fill_i32(p, 0, n, s);
}

void label_sort_reset_region(void* ws, int64_t B, int64_t N, int64_t K,
                             int32_t** p, int64_t* n) {
  *p = nullptr;
  *n = 0;
  if (B == 0 || N == 0) return;
  SortBufs w = carve_sort(ws, B, N, K, nullptr);
  *p = w.err;
  *n = w.nctl;
}

}  // namespace fkc
