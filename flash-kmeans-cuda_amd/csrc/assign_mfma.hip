// Fused distance + argmin on gfx950 matrix cores (fp16 / bf16 inputs).
//
// What it computes (same ranking as the reference's raw-distance MMA route,
// flash_kmeans_cuda/csrc/assign/assign_sm80.cu:437-441 with RAW_DIST=true at
// :687): for every point n of batch b,
//     ids[b,n] = argmax_k ( <x_n, c_k> - c_sq[k]/2 )
//              = argmin_k ( c_sq[k] - 2 <x_n, c_k> ),
// the lowest k winning exact ties (assign_common.cuh:20-28,
// assign_sm80.cu:594-611).  x_sq is row-constant for the argmin and is not
// read.  Products are exact in fp32 and accumulate in fp32 (the reference
// accumulates fp16 inputs in fp16, assign_sm80.cu:81-118).
//
// Mapping onto v_mfma_f32_16x16x32_{f16,bf16} (D = A*B + C, 16x16 tiles,
// 32 features per step):
//   A (rows)    = 16 centroids x 32 features, streamed through LDS;
//   B (columns) = 32 features x 16 points, held in VGPRs for the whole K
//                 loop (lane l owns point l%16, features 8(l/16)..+7 of each
//                 32-feature step);
//   C           = -c_sq/2 of the 16 centroids, so the accumulator leaves the
//                 matrix core holding the score to maximise; centroids past K
//                 get -inf and can never win.
// Lane l holds column (point) l%16 and rows 4(l/16)+r, r = 0..3: four scores
// of one point against consecutive centroids.  A lane keeps its best score
// and the 16-centroid block where it first appeared (two max3 and a
// compare-select per four scores, branch-free, so the vector ALU stays well
// under the matrix core's time per score and the next block's MFMA chain
// issues under this block's fold).  At the end the four lanes that share a
// point (l, l+16, l+32, l+48) merge with the lowest-index rule, and the
// winner's four candidate rows are scored again by the same MFMA chain to
// pick the first maximal one.  For K <= FKC_EXACT_MAX_K (512) the loop
// tracks the exact index instead (the re-score would cost more than it
// saves).  Where a launch runs at most two waves per SIMD (grids of <= 512
// four-tile workgroups at D = 97..128) the loop also keeps each lane's
// scores of its best block, so no re-score is needed at all.
// Feature widths that are not a multiple of 32 are zero-padded in registers
// and LDS (zeros add nothing to a dot product).
//
// Workgroup: 4 waves x PT point tiles x 16 points (PT chosen per grid size;
// PT = 8 at D = 128 on large grids: 128 point registers, 2 waves per SIMD).
// Centroids pass through LDS in double-buffered stages with one barrier per
// stage; the next stage's loads are in flight while the matrix cores work
// on the current one.  For D = 32, 64, 128 and 256 the stages are direct
// global->LDS loads into unpadded, XOR-permuted rows (no staging registers,
// no bank conflicts); other widths stage through VGPRs into rows padded by
// 16 bytes.
// Centroid rows past K re-read row K-1 instead of branching (their scores
// are masked to -inf).
// Where a batch row's whole centroid table fits one workgroup's LDS (D = 32
// and 64, K up to 2400 / 1216) and the grid gives every CU a workgroup,
// assign_resident_kernel loads the table once per workgroup and its 16
// waves walk their point tiles against it with no barrier in the loop; its
// scores and fold are the same, so its labels are identical.
#include "device_util.hpp"
#include "fkc_internal.hpp"

#include <hip/hip_ext.h>

#include <algorithm>
#include <atomic>
#include <math.h>

namespace fkc {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Compile-time tunables (defaults measured on MI355X at the benchmark
// shapes): FKC_AB, minimum waves per SIMD asked of the register allocator
// for the lighter variants (D = 33..64 asks 4: its four-tile variant then
// fits 120 VGPRs instead of 129, 4 waves per SIMD instead of 3, and the c4
// grid of 2048 workgroups runs in 2 rounds instead of 2.67: 101.8 -> 91.6
// us at (8, 65536, 1024, 64) bf16; at D = 32 the same bound cost 5%);
// FKC_EXACT_MAX_K (FKC_EXACT_MAX_K_NARROW at D <= 64), largest K that
// tracks the exact index in the loop; FKC_USE_DMA, direct global->LDS
// stages where eligible;
// FKC_KC_DMA, centroid rows per direct stage at D = 97..128 (x4 at D = 32,
// x2 at D = 64); FKC_KC_DMA8, the
// same for the eight-tile variant (two workgroups per CU leave it twice the
// LDS; at c5, bench defaults, same box: 128 rows 0.795 / 0.797 ms per
// iteration, 144 rows 0.798 / 0.799 (four registers spilled), 96 rows
// 0.799 / 0.801); FKC_SLICE_MIN_ROWS, the shortest centroid slice; FKC_SCHED_GROUPS,
// LDS-read / MFMA / VALU ordering hints in the direct-stage loop.
#ifndef FKC_AB
#define FKC_AB 2
#endif
#ifndef FKC_EXACT_MAX_K
#define FKC_EXACT_MAX_K 512
#endif
#ifndef FKC_EXACT_MAX_K_NARROW
#define FKC_EXACT_MAX_K_NARROW 512
#endif
#ifndef FKC_USE_DMA
#define FKC_USE_DMA 1
#endif
#ifndef FKC_KC_DMA
#define FKC_KC_DMA 64
#endif
#ifndef FKC_KC_DMA8
#define FKC_KC_DMA8 128
#endif
#ifndef FKC_KC_DMA_SAVE
#define FKC_KC_DMA_SAVE 128
#endif
#ifndef FKC_SLICE_MIN_ROWS
#define FKC_SLICE_MIN_ROWS 2048
#endif
#ifndef FKC_SCHED_GROUPS
#define FKC_SCHED_GROUPS 1
#endif
// FKC_X_NT=1: point rows are loaded with the non-temporal hint.  Each point
// row is read by one workgroup, once, so the assign itself gains nothing
// from caching it, and without the hint the streaming rows evict centroid
// stages from L2 (c5: 186 MB fetched per launch against 138 MB of
// algorithmic bytes; with the hint 154 MB, same assign time).  Off by
// default: the Lloyd iteration then ran 6-7 us slower at c5 (0.797 against
// 0.790 ms, same box, alternating runs), the update's gathers of the same
// rows finding fewer of them in the device's last-level cache.
#ifndef FKC_X_NT
#define FKC_X_NT 0
#endif
// FKC_WHOLE_STAGE=0 (compile time, for A/B builds) keeps small exact-index
// tables on the double-buffered 64-row stages.
#ifndef FKC_WHOLE_STAGE
#define FKC_WHOLE_STAGE 1
#endif

constexpr int KC = 64;  // centroid rows per register-staged LDS stage
constexpr int THREADS = 256;  // 4 waves

template <int DT>
__device__ inline f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c);

template <>
__device__ inline f32x4 mfma16<FKC_F16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(
      __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <>
__device__ inline f32x4 mfma16<FKC_BF16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
      __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
      0);
}

// Slot permutation of unpadded stage rows: row r keeps feature segment v in
// slot v ^ swz(r).  Sixteen consecutive rows (one fragment read) then cover
// 16 distinct 16-byte bank groups for any SEGS = 4, 8, 16, 32.
template <int SEGS>
__device__ constexpr int swz(int r) {
  return SEGS >= 16 ? (r & 15) : ((r & 15) / (16 / SEGS));
}

// One 16-byte piece of a point row (see FKC_X_NT).
__device__ inline u32x4 load_point(const u32x4* p) {
#if FKC_X_NT
  return __builtin_nontemporal_load(p);
#else
  return *p;
#endif
}

// Running maximum of a lane's scores.  The main loop keeps, per lane and
// point tile, only the best score and the first 16-centroid block that
// reached it (a wave-uniform value): two max3 and a compare-select per four
// scores, with no branch, so the matrix-core chain of the next block can
// issue under the fold of this one.  Which of the lane's four rows in that
// block won is settled once at the end.
__device__ inline void fold_block(const f32x4& acc, float& best, int& bblk,
                                  int blk) {
  const float nb = fmaxf(fmaxf(fmaxf(fmaxf(best, acc[0]), acc[1]), acc[2]),
                         acc[3]);
  bblk = nb > best ? blk : bblk;  // strict: equal later scores keep the first
  best = nb;
}

// Exact running (best, index) over a lane's four scores of block rows
// kt..kt+3, the first maximal row winning; used when K is small, where the
// end-of-loop recompute would cost more than it saves.
__device__ inline void fold_exact(const f32x4& acc, float& best, int& bidx,
                                  int kt) {
  const float nb = fmaxf(fmaxf(fmaxf(fmaxf(best, acc[0]), acc[1]), acc[2]),
                         acc[3]);
  const int j = acc[0] == nb ? 0 : (acc[1] == nb ? 1 : (acc[2] == nb ? 2 : 3));
  bidx = nb > best ? kt + j : bidx;
  best = nb;
}

// Block fold that also keeps the lane's four scores of the block where its
// running maximum was first reached, so the winning row is known at the end
// without re-scoring: the first of the four saved scores equal to the best.
// Four register selects per four scores more than fold_block; used where
// the grid leaves registers spare (two waves per SIMD).
__device__ inline void fold_saved(const f32x4& acc, float& best, int& bblk,
                                  f32x4& saved, int blk) {
  const float nb = fmaxf(fmaxf(fmaxf(fmaxf(best, acc[0]), acc[1]), acc[2]),
                         acc[3]);
  const bool up = nb > best;  // strict: equal later scores keep the first
  bblk = up ? blk : bblk;
#pragma unroll
  for (int j = 0; j < 4; ++j) saved[j] = up ? acc[j] : saved[j];
  best = nb;
}

// Issue priority by progress: 3 in the first quarter of a workgroup's
// stages, then 2, 1, 0.  Two workgroups share each SIMD of a CU, and the
// arbiter prefers the older wave: without this the one that started first
// ran ahead (c3: its loop 44 us against 57 us for its partner on every CU;
// c5: 266 against 392 us) and the other finished alone, one wave per SIMD
// with nothing to hide its latency.  With priority falling as a workgroup
// advances, the one behind wins arbitration, so the pair stays level.
__device__ inline void progress_prio(int done, int total) {
  const int q = (4 * done) / total;  // 0..3 while done < total
  if (q == 0)
    __builtin_amdgcn_s_setprio(3);
  else if (q == 1)
    __builtin_amdgcn_s_setprio(2);
  else if (q == 2)
    __builtin_amdgcn_s_setprio(1);
  else
    __builtin_amdgcn_s_setprio(0);
}

// DS2: 32-feature steps (padded width DP = 32*DS2 >= D); PT: 16-point tiles
// per wave; PAD: D < DP, so segments past D read as zeros (a compile-time
// flag: the unpadded variants carry no per-load condition); EXACT: track
// the exact index in the loop instead of re-scoring at the end; SAVE: keep
// the best block's scores (fold_saved) instead of re-scoring at the end
// (two waves per SIMD, 128-row stages); WHOLE (exact index, direct stages):
// the table in one single-buffered stage of up to 256 rows (64 KB at
// D = 128), loaded in one round trip with one barrier, where the
// double-buffered 64-row stages take one round trip each.  D % 8 == 0 so
// every 8-feature segment is a 16-byte load.
template <int DT, int DS2, int PT, bool PAD, bool EXACT, bool SAVE,
          bool WHOLE = false>
__global__ void __launch_bounds__(THREADS,
                                  PT == 8 ? 2
                                  : (SAVE && DS2 == 2) ? 3
                                  : (DS2 == 2 && PT <= 4) ? 4
                                  : (PT * DS2 <= 16 && DS2 <= 9) ? FKC_AB
                                                                 : 1)
assign_mfma_kernel(const uint16_t* __restrict__ x,
                   const uint16_t* __restrict__ cent,
                   const float* __restrict__ c_sq, int32_t* __restrict__ ids,
                   int N, int K, int D, const int32_t* __restrict__ ctrl,
                   int kspan, float* __restrict__ psc,
                   int32_t* __restrict__ pidx) {
  if (loop_done(ctrl)) return;
  // Centroid slice (grid z): rows k0 .. k0 + kspan - 1 of the batch's K,
  // scored below as a problem of K' = min(K - k0, kspan) rows.  With one
  // slice the winner goes to ids; with several, each slice writes its
  // winner's score and row to psc / pidx and assign_merge_kernel picks the
  // first maximum in slice order (the slices' scores are the same MFMA
  // chains as unsliced, so the labels are identical).
  const int Kall = K;
  const int k0 = blockIdx.z * kspan;
  K = min(Kall - k0, kspan);
  constexpr int DP = DS2 * 32;
  constexpr int ROW = DP + 8;       // LDS row stride in 16-bit elements
  constexpr int SEGS = DP / 8;      // 16-byte segments per padded row
  constexpr int PIECES = KC * SEGS;
  constexpr int PPT = (PIECES + THREADS - 1) / THREADS;
  constexpr int PTS_WAVE = PT * 16;
  constexpr int PTS_WG = 4 * PTS_WAVE;
  constexpr int NT = KC / 16;

  // Direct-to-LDS stages for unpadded power-of-two step counts (D = 32, 64,
  // 128, 256); measured faster than register staging at D = 64 and 128.
  constexpr bool DMA =
      FKC_USE_DMA && !PAD && (DS2 == 1 || DS2 == 2 || DS2 == 4 || DS2 == 8);

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, g = lane >> 4;
  const int b = blockIdx.y;
  const int dsegs = D / 8;          // real segments per row
  constexpr bool padded = PAD;
  const uint16_t* xb = x + (size_t)b * N * D;
  const uint16_t* cb = cent + ((size_t)b * Kall + k0) * D;
  const float* qb = c_sq + (size_t)b * Kall + k0;
  const int n0 = blockIdx.x * PTS_WG + wave * PTS_WAVE;

  // B operand: point n0+16p+col, features 32s + 8g .. +7.  Points past N
  // load point N-1 (their labels are not stored).
  u32x4 xr[PT][DS2];
#pragma unroll
  for (int p = 0; p < PT; ++p) {
    const int n = min(n0 + 16 * p + col, N - 1);
    const u32x4* src = reinterpret_cast<const u32x4*>(xb + (size_t)n * D);
#pragma unroll
    for (int s = 0; s < DS2; ++s) {
      const int seg = 4 * s + g;
      xr[p][s] = (!padded || seg < dsegs) ? load_point(src + seg)
                                          : u32x4{0u, 0u, 0u, 0u};
    }
  }

  float best[PT];
  int bblk[PT];
  f32x4 sv[SAVE ? PT : 1];  // SAVE: the lane's scores of its best block
#pragma unroll
  for (int p = 0; p < PT; ++p) {
    best[p] = -INFINITY;
    bblk[p] = 0;
    if constexpr (SAVE) sv[p] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  }

  // Fold one 16-centroid block's accumulators into the running maxima.
  auto fold = [&](const f32x4* acc, int blk) {
#pragma unroll
    for (int p = 0; p < PT; ++p) {
      if constexpr (EXACT)
        fold_exact(acc[p], best[p], bblk[p], blk + 4 * g);
      else if constexpr (SAVE)
        fold_saved(acc[p], best[p], bblk[p], sv[SAVE ? p : 0], blk);
      else
        fold_block(acc[p], best[p], bblk[p], blk);
    }
  };

  if constexpr (DMA) {
    // Direct global->LDS stages (buffer loads with the LDS bit).  A wave's
    // load instruction writes 64 lanes x 16 bytes to consecutive LDS, so a
    // stage row is stored unpadded as SEGS 16-byte slots, slot v holding
    // feature segment v ^ swz(row): the sixteen rows a fragment read touches
    // then fall on distinct banks.  The two stage buffers are separate
    // arrays, so the compiler can tell that loads into one do not alias
    // reads from the other.  Each stage is addressed through a buffer
    // resource built from its wave-uniform base (scalar registers) plus a
    // fixed 32-bit per-lane offset, so a stage's loads cost no vector ALU
    // work and hold no 64-bit addresses in VGPRs.  Buffer (not global)
    // loads also let the compiler wait for LDS reads by count while the
    // next stage's loads are in flight; with global loads to LDS it waits
    // for every outstanding LDS read at each use.  With K >= KCD no row is
    // clamped: the last stage starts at K - KCD instead, re-scoring rows an
    // earlier stage saw (a re-seen row can never beat its own earlier
    // score, so the first-maximum rule still holds, and every candidate row
    // stays below K).  Only K < KCD clamps rows to K-1.  c_sq lands raw and
    // each wave scales (and masks past K) its own share once its loads are
    // in, before the barrier.
    // Stage rows: FKC_KC_DMA rows at D = 97..128; the narrow widths keep
    // the same 16 KB per stage with more rows (D = 32: 256 rows, 0.026 ->
    // 0.021 ms at (2, 30000, 2000, 32); D = 64: 128 rows, ~1%), so a stage
    // still spans enough matrix work to hide its barrier.
    constexpr int KCD0 = WHOLE      ? (DS2 <= 4 ? 256 : 128)
                         : PT == 8    ? FKC_KC_DMA8
                         : SAVE     ? FKC_KC_DMA_SAVE
                         : DS2 == 1 ? 4 * FKC_KC_DMA
                         : DS2 == 2 ? 2 * FKC_KC_DMA
                         : DS2 <= 4 ? FKC_KC_DMA
                                    : 64;
    constexpr int KCD = (KCD0 * DP * 2) % (THREADS * 16) == 0 ? KCD0 : 64;
    constexpr int ROWB = DP * 2;
    constexpr int STAGE = KCD * ROWB;
    constexpr int LOADS = STAGE / (THREADS * 16);
    constexpr int QW = KCD / 4;  // c_sq entries loaded per wave
    constexpr int RSRC_W3 = 0x00020000;  // buffer resource word 3 (gfx9)
    static_assert(STAGE % (THREADS * 16) == 0 && QW <= 64, "stage split");
    static_assert((ROWB & (ROWB - 1)) == 0, "power-of-two stage rows");
    __shared__ __attribute__((aligned(1024))) uint8_t s_c0[STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t s_c1[WHOLE ? 16 : STAGE];
    __shared__ __attribute__((aligned(256))) float s_q0[KCD];
    __shared__ __attribute__((aligned(256))) float s_q1[WHOLE ? 4 : KCD];
    typedef __attribute__((address_space(3))) void lvoid;

    const int uwave = __builtin_amdgcn_readfirstlane(wave);  // scalar copy
    const int nch = (K + KCD - 1) / KCD;
    const bool overlap = K >= KCD;     // wave-uniform
    // Source byte of load j within a stage: row * ROWB + permuted segment
    // (rows clamped to K-1 when K < KCD).
    uint32_t so[LOADS];
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const int pos = (uwave * LOADS + j) * 1024 + lane * 16;
      const int r = pos / ROWB, v = (pos % ROWB) / 16;
      so[j] = (uint32_t)((overlap ? r : min(r, K - 1)) * ROWB +
                         (v ^ swz<SEGS>(r)) * 16);
    }
    const int qi = uwave * QW + lane;  // this lane's c_sq slot (lane < QW)
    const uint32_t qo = (uint32_t)(overlap ? qi : min(qi, K - 1)) * 4;
    const int sw = swz<SEGS>(col);     // rows 16t + col share it
    const char* cbase = reinterpret_cast<const char*>(cb);
    auto kbase = [&](int chunk) {      // first centroid row of a stage
      return __builtin_amdgcn_readfirstlane(
          overlap ? min(chunk * KCD, K - KCD) : 0);
    };

    // (The offsets are passed through locals: with a captured variable as
    // the offset argument this clang emits no host launch stub for the
    // kernel.)
    auto issue = [&](int chunk, uint8_t* dc, float* dq) {
      const int kb = kbase(chunk);
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(cbase + (size_t)kb * ROWB), 0, STAGE, RSRC_W3);
#pragma unroll
      for (int j = 0; j < LOADS; ++j) {
        const uint32_t off = so[j];
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (lvoid*)(dc + (uwave * LOADS + j) * 1024), 16, off, 0, 0, 0);
      }
      if (lane < QW) {
        const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(qb + kb), 0, KCD * 4, RSRC_W3);
        const uint32_t off = qo;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rq, (lvoid*)(dq + uwave * QW), 4, off, 0, 0, 0);
      }
    };
    // After this wave's loads have landed: scale its c_sq share in place.
    // Branch-free (the 64 / QW lanes that share an entry write the same
    // value), so no block boundary splits the stage's code: a boundary here
    // lets the compiler sink the stage's folds below it, away from the
    // matrix-core work they should overlap.
    const int qf = uwave * QW + (lane % QW);
    auto fixq = [&](int chunk, float* dq) {
      const int k = kbase(chunk) + qf;
      const float v = dq[qf];
      dq[qf] = k < K ? -0.5f * v : -INFINITY;
    };
    auto frag = [&](const uint8_t* lc, const float* lq, int t, u32x4* a,
                    f32x4& ci) {
      ci = *reinterpret_cast<const f32x4*>(lq + 16 * t + 4 * g);
      const uint8_t* arow = lc + (16 * t + col) * ROWB;
#pragma unroll
      for (int s = 0; s < DS2; ++s)
        a[s] = *reinterpret_cast<const u32x4*>(arow + (((4 * s + g) ^ sw) * 16));
    };
    // Software-pipelined over the stage's 16-centroid blocks: the fragments
    // of block t+1 are read from LDS while block t is on the matrix core,
    // and block t-1 is folded on the vector ALU under block t's MFMAs.  For
    // four point tiles the scheduling groups fix that order (LDS reads for
    // the next block first, then MFMA / VALU alternating) rather than let
    // the compiler issue the whole stage's MFMAs first and its folds last,
    // which keeps every accumulator alive at once and serialises the two
    // units within a wave, or read each fragment just before its MFMA,
    // which exposes the LDS latency every 4 MFMAs (measured at N=524288,
    // K=8192, D=128: 0.86 -> 0.81 ms for the MFMA/VALU groups, a further
    // 0.79 -> 0.76 ms for the read-ahead; with fewer tiles the groups cost
    // time).
    auto compute = [&](int chunk, const uint8_t* lc, const float* lq) {
      const int kb = kbase(chunk);
      constexpr int NTD = KCD / 16;
      if constexpr (EXACT) {
        // Small K: few stages, so no pipelining; blocks wholly past K (a
        // partial last stage) are skipped.
#pragma unroll
        for (int t = 0; t < NTD; ++t) {
          if (kb + 16 * t >= K) break;
          u32x4 a[DS2];
          f32x4 ci;
          frag(lc, lq, t, a, ci);
          f32x4 acc[PT];
#pragma unroll
          for (int s = 0; s < DS2; ++s) {
#pragma unroll
            for (int p = 0; p < PT; ++p)
              acc[p] = mfma16<DT>(a[s], xr[p][s], s == 0 ? ci : acc[p]);
          }
          fold(acc, kb + 16 * t);
        }
      } else if constexpr (PT == 8) {
        // Eight tiles: the point registers leave no room for a second set
        // of accumulators, so each block is folded after its own MFMAs; the
        // next block's fragments are still read a block ahead, and the
        // compiler overlaps one block's folds with the next block's matrix
        // work (measured at N=524288, K=8192, D=128: 0.784 -> 0.749 ms
        // against four tiles, from half the LDS fragment reads and half the
        // centroid stage traffic per point).
        u32x4 an[DS2];
        f32x4 cn;
        frag(lc, lq, 0, an, cn);
#pragma unroll
        for (int t = 0; t < NTD; ++t) {
          u32x4 a[DS2];
          f32x4 ci = cn;
#pragma unroll
          for (int s = 0; s < DS2; ++s) a[s] = an[s];
          if (t + 1 < NTD) frag(lc, lq, t + 1, an, cn);
          f32x4 acc[PT];
#pragma unroll
          for (int s = 0; s < DS2; ++s) {
#pragma unroll
            for (int p = 0; p < PT; ++p)
              acc[p] = mfma16<DT>(a[s], xr[p][s], s == 0 ? ci : acc[p]);
          }
          fold(acc, kb + 16 * t);
        }
      } else {
        f32x4 prev[PT];
        u32x4 an[DS2];  // fragments of the next block
        f32x4 cn;
        frag(lc, lq, 0, an, cn);
#pragma unroll
        for (int t = 0; t < NTD; ++t) {
          u32x4 a[DS2];
          f32x4 ci = cn;
#pragma unroll
          for (int s = 0; s < DS2; ++s) a[s] = an[s];
          if (t + 1 < NTD) frag(lc, lq, t + 1, an, cn);
          f32x4 acc[PT];
#pragma unroll
          for (int s = 0; s < DS2; ++s) {
#pragma unroll
            for (int p = 0; p < PT; ++p)
              acc[p] = mfma16<DT>(a[s], xr[p][s], s == 0 ? ci : acc[p]);
          }
          if (t > 0) fold(prev, kb + 16 * (t - 1));
          if constexpr (FKC_SCHED_GROUPS && PT >= 4) {
            // Block 0 also takes block 1's reads (a stage's first two
            // blocks are read back to back after the barrier).
            if (t == 0 && NTD > 1)
              __builtin_amdgcn_sched_group_barrier(0x100, 2 * (DS2 + 1), 0);
            else if (t + 1 < NTD)
              __builtin_amdgcn_sched_group_barrier(0x100, DS2 + 1, 0);
#pragma unroll
            for (int i = 0; i < DS2 * PT; ++i) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
              __builtin_amdgcn_sched_group_barrier(0x002, SAVE ? 2 : 1, 0);  // VALU
            }
          }
#pragma unroll
          for (int p = 0; p < PT; ++p) prev[p] = acc[p];
        }
        fold(prev, kb + 16 * (NTD - 1));
      }
    };

    // The wait for the next stage's loads stays at the end of the stage:
    // the scheduling barrier keeps the compiler from hoisting it above the
    // stage's matrix work.
    if constexpr (WHOLE) {
      // One buffer (the plan takes this variant where the table is one
      // stage; more stages run one after the other).
      for (int chunk = 0; chunk < nch; ++chunk) {
        if (chunk > 0) __syncthreads();  // the previous stage is read
        issue(chunk, s_c0, s_q0);
        __builtin_amdgcn_s_waitcnt(0);
        fixq(chunk, s_q0);
        __syncthreads();
        compute(chunk, s_c0, s_q0);
      }
    } else {
    issue(0, s_c0, s_q0);
    __builtin_amdgcn_s_waitcnt(0);
    fixq(0, s_q0);
    __syncthreads();
    for (int chunk = 0; chunk < nch; chunk += 2) {
      progress_prio(chunk, nch);
      if (chunk + 1 < nch) issue(chunk + 1, s_c1, s_q1);
      compute(chunk, s_c0, s_q0);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(0);
      fixq(chunk + 1, s_q1);  // harmless on a stage that was not loaded
      __syncthreads();
      if (chunk + 1 >= nch) break;
      if (chunk + 2 < nch) issue(chunk + 2, s_c0, s_q0);
      compute(chunk + 1, s_c1, s_q1);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(0);
      fixq(chunk + 2, s_q0);
      __syncthreads();
    }
    }
  } else {
    // Stages through VGPRs into padded LDS rows (row stride DP + 8 halves).
    __shared__ __attribute__((aligned(16))) uint16_t lds_c[2][KC * ROW];
    __shared__ __attribute__((aligned(16))) float lds_q[2][KC];
    u32x4 pf[PPT];
    float pq = 0.f;  // raw c_sq of the prefetched stage (scaled when stored)
    const int nchunks = (K + KC - 1) / KC;

    auto gload = [&](int chunk) {
      const int kb = chunk * KC;
  #pragma unroll
      for (int j = 0; j < PPT; ++j) {
        const int i = tid + j * THREADS;
        if (PIECES % THREADS == 0 || i < PIECES) {
          const int r = i / SEGS, sg = i % SEGS;
          const int k = min(kb + r, K - 1);
          const u32x4* row = reinterpret_cast<const u32x4*>(cb + (size_t)k * D);
          pf[j] = (!padded || sg < dsegs) ? row[sg] : u32x4{0u, 0u, 0u, 0u};
        }
      }
      // Only the load is issued here; using the value (scale, mask) waits for
      // it, which would stall this wave before the stage's matrix work.  All
      // threads load (four per entry), so no branch splits the stage's code.
      pq = qb[min(kb + (tid & (KC - 1)), K - 1)];
    };
    auto lstore = [&](int buf, int chunk) {
      const int kb = chunk * KC;
  #pragma unroll
      for (int j = 0; j < PPT; ++j) {
        const int i = tid + j * THREADS;
        if (PIECES % THREADS == 0 || i < PIECES) {
          const int r = i / SEGS, sg = i % SEGS;
          *reinterpret_cast<u32x4*>(&lds_c[buf][r * ROW + sg * 8]) = pf[j];
        }
      }
      const int k = kb + (tid & (KC - 1));
      lds_q[buf][tid & (KC - 1)] = k < K ? -0.5f * pq : -INFINITY;
    };

    gload(0);
    lstore(0, 0);
    __syncthreads();

    for (int chunk = 0; chunk < nchunks; ++chunk) {
      const int buf = chunk & 1;
      progress_prio(chunk, nchunks);
      if (chunk + 1 < nchunks) gload(chunk + 1);
      const uint16_t* lc = lds_c[buf];
      const float* lq = lds_q[buf];
      auto tile = [&](int t, f32x4* acc) {
        const f32x4 cinit = *reinterpret_cast<const f32x4*>(lq + 16 * t + 4 * g);
        const u32x4* arow =
            reinterpret_cast<const u32x4*>(lc + (16 * t + col) * ROW) + g;
        u32x4 a[DS2];
#pragma unroll
        for (int s = 0; s < DS2; ++s) a[s] = arow[4 * s];
#pragma unroll
        for (int s = 0; s < DS2; ++s) {
#pragma unroll
          for (int p = 0; p < PT; ++p)
            acc[p] = mfma16<DT>(a[s], xr[p][s], s == 0 ? cinit : acc[p]);
        }
      };
      // (Folding block t-1 under block t, as the direct-stage path does,
      // measured no faster here.)
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        f32x4 acc[PT];
        tile(t, acc);
        fold(acc, chunk * KC + 16 * t);
      }
      // Unconditional (after the last stage it fills the idle buffer with
      // data nobody reads), so no branch splits the stage's code.
      lstore(buf ^ 1, chunk + 1);
      __syncthreads();
    }
  }

  // Settle each point: the four lanes sharing it (g = 0..3) hold the best
  // score of their rows and the block where it first appeared; the winner
  // is the higher score, ties to the lower candidate base blk + 4g (the four
  // candidate ranges do not interleave).  Then the four candidates
  // base + r are scored again with the same instruction, operands and
  // accumulator seed as in the loop, one MFMA chain per r with row i holding
  // point i's candidate, and the first r reaching the maximum of the
  // diagonal wins.
  if constexpr (EXACT) {
#pragma unroll
    for (int p = 0; p < PT; ++p) {
      float bv = best[p];
      int bi = bblk[p];
#pragma unroll
      for (int off = 16; off <= 32; off <<= 1) {
        const float ob = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (ob > bv || (ob == bv && oi < bi)) {
          bv = ob;
          bi = oi;
        }
      }
      const int n = n0 + 16 * p + col;
      if (g == 0 && n < N) {
        if (psc != nullptr) {
          const size_t o = ((size_t)b * gridDim.z + blockIdx.z) * N + n;
          psc[o] = bv;
          pidx[o] = k0 + bi;
        } else {
          ids[(size_t)b * N + n] = bi;
        }
      }
    }
    return;
  }
  if constexpr (SAVE) {
    // The winning row of each lane is the first of its saved scores equal
    // to its best; the four lanes of a point then keep the higher score,
    // ties to the lower row (lane rows do not interleave within a block, and
    // an earlier block has lower rows).  min() only guards degenerate input
    // (every score -inf or NaN): the label stays a valid row.
#pragma unroll
    for (int p = 0; p < PT; ++p) {
      float bv = best[p];
      const f32x4 v = sv[SAVE ? p : 0];
      const int j = v[0] == bv ? 0 : (v[1] == bv ? 1 : (v[2] == bv ? 2 : 3));
      int bi = min(bblk[p] + 4 * g + j, K - 1);
#pragma unroll
      for (int off = 16; off <= 32; off <<= 1) {
        const float ob = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (ob > bv || (ob == bv && oi < bi)) {
          bv = ob;
          bi = oi;
        }
      }
      const int n = n0 + 16 * p + col;
      if (g == 0 && n < N) {
        if (psc != nullptr) {
          const size_t o = ((size_t)b * gridDim.z + blockIdx.z) * N + n;
          psc[o] = bv;
          pidx[o] = k0 + bi;
        } else {
          ids[(size_t)b * N + n] = bi;
        }
      }
    }
    return;
  }
#pragma unroll
  for (int p = 0; p < PT; ++p) {
    float bv = best[p];
    int base = bblk[p] + 4 * g;
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1) {
      const float ob = __shfl_xor(bv, off, 64);
      const int obase = __shfl_xor(base, off, 64);
      if (ob > bv || (ob == bv && obase < base)) {
        bv = ob;
        base = obase;
      }
    }
    // Every load of the re-score is issued before any of them is used:
    // unconditional, from rows clamped to K - 1 (a clamped row only stands
    // for a candidate past K, whose seed is -inf below), so the tile costs
    // one memory round trip rather than one per load.  Each lane loads its
    // own point's four candidate rows (its segments of them) and their c_sq.
    float cq[4];
    u32x4 ar[4][DS2];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int kr = min(base + r, K - 1);
      cq[r] = qb[kr];
      const u32x4* crow = reinterpret_cast<const u32x4*>(cb + (size_t)kr * D);
#pragma unroll
      for (int s = 0; s < DS2; ++s) {
        const int seg = 4 * s + g;
        // Padded widths load an in-bounds segment and zero it past D.
        const u32x4 v = crow[padded ? min(seg, dsegs - 1) : seg];
        ar[r][s] = (!padded || seg < dsegs) ? v : u32x4{0u, 0u, 0u, 0u};
      }
    }
    // Only the diagonal of each chain is read: accumulator row i = col
    // (element e = col & 3 of the lane with g == col / 4) is point col
    // against its own candidate, and that lane loaded this very point's
    // base and candidate c_sq.  So every lane seeds all four rows with its
    // own point's value: the diagonal gets the loop's seed, the rest is
    // never read (no cross-lane exchange of bases or c_sq is needed).
    const int e = col & 3;  // this lane's diagonal element when g == col/4
    float dv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float seed = base + r < K ? -0.5f * cq[r] : -INFINITY;
      f32x4 acc = {seed, seed, seed, seed};
#pragma unroll
      for (int s = 0; s < DS2; ++s) acc = mfma16<DT>(ar[r][s], xr[p][s], acc);
      float d = acc[0];
      d = e == 1 ? acc[1] : d;
      d = e == 2 ? acc[2] : d;
      d = e == 3 ? acc[3] : d;
      dv[r] = d;
    }
    int rr = 0;
    float m = dv[0];
#pragma unroll
    for (int r = 1; r < 4; ++r) {
      if (dv[r] > m) {
        m = dv[r];
        rr = r;
      }
    }
    const int n = n0 + 16 * p + col;
    if (g == (col >> 2) && n < N) {
      if (psc != nullptr) {
        const size_t o = ((size_t)b * gridDim.z + blockIdx.z) * N + n;
        psc[o] = m;
        pidx[o] = k0 + base + rr;
      } else {
        ids[(size_t)b * N + n] = base + rr;
      }
    }
  }
}

// Merge of centroid slices: per point, the first slice (lowest rows) with
// the maximal score wins, and within a slice the kernel already kept the
// first maximal row, so the label is the lowest index of the maximum, as
// unsliced.
__global__ void __launch_bounds__(256)
assign_merge_kernel(const float* __restrict__ psc,
                    const int32_t* __restrict__ pidx, int32_t* __restrict__ ids,
                    int N, int S, const int32_t* __restrict__ ctrl) {
  if (loop_done(ctrl)) return;
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  const size_t b = blockIdx.y;
  const size_t o = b * S * N + n;
  float best = psc[o];
  int bi = pidx[o];
  for (int z = 1; z < S; ++z) {
    const float v = psc[o + (size_t)z * N];
    const int i = pidx[o + (size_t)z * N];
    bi = v > best ? i : bi;
    best = fmaxf(best, v);
  }
  ids[b * N + n] = bi;
}

// ------------------------------------------------------------------------
// Centroid-resident variant.  When a batch row's whole centroid table fits
// in one workgroup's LDS (Kp = K rounded up to 32 rows of DP features, plus
// Kp scaled c_sq values and a little padding: resident_bytes(Kp) <= the
// device's LDS per
// workgroup, i.e. on gfx950's 160 KiB K <= 1216 at D = 64 and K <= 2400 at
// D = 32), each workgroup loads the table once
// and its waves then walk their 16*PT-point tiles against it on their own:
// no stage loads or barriers in the loop, the winner's candidate rows are
// scored again from LDS rather than L2, and a wave that is loading its next
// points or settling its labels leaves the matrix core to the other waves
// of its SIMD instead of idling it for a whole round of workgroups.  The
// scores are the same MFMA chains with the same seeds as the staged kernel,
// folded by the same block rule and re-score, so the labels are identical.
// The table's LDS bound is the device's per-workgroup LDS (160 KiB on
// gfx950, read with the CU count by device_shape()).
constexpr int kResidentWaves = 16;        // waves per workgroup (4 per SIMD)

// The table, its scaled c_sq, and room for the loop's fragment read one
// block past the table (rows Kp .. Kp + 15 and c_sq entries Kp .. Kp + 15,
// read in the last trip and never used): the rows fall on the c_sq region
// and past it by 16 rows' bytes less that region, the c_sq entries 64 bytes
// past it.
__host__ __device__ constexpr int resident_bytes(int ds2, int Kp) {
  return Kp * (ds2 * 64 + 4) +
         (16 * ds2 * 64 > 4 * Kp ? 16 * ds2 * 64 - 4 * Kp : 0) + 64;
}

// W waves per workgroup, PT tiles per wave: 16 x 8 at D = 32 (a block's
// fragment read then feeds eight MFMAs, as at D = 64 with four) and 16 x 4
// at D = 64, both within 128 VGPRs (4 waves per SIMD).  Measured at
// (8, 65536, 1024, 64) bf16 against the staged kernel's 0.067-0.070 ms:
// 0.063 ms (the loop unrolled by two so the fragment and accumulator sets
// rotate without copies; 0.076 with a copy per block), progress priorities
// 4.6% fewer cycles (matrix core busy 46.8 -> 49.1%, 2.59 -> 3.06 waves
// resident per SIMD).  Eight tiles on eight waves at D = 64 (half the
// fragment reads per MFMA at 2 waves per SIMD) and issue priorities
// staggered over a SIMD's waves measured no faster.
template <int DT, int DS2, int PT, int W>
__global__ void __launch_bounds__(W * 64, 1)
assign_resident_kernel(const uint16_t* __restrict__ x,
                       const uint16_t* __restrict__ cent,
                       const float* __restrict__ c_sq,
                       int32_t* __restrict__ ids, int N, int K,
                       const int32_t* __restrict__ ctrl) {
  if (loop_done(ctrl)) return;
  constexpr int DP = DS2 * 32;
  constexpr int ROWB = DP * 2;
  constexpr int SEGS = DP / 8;
  constexpr int NTH = W * 64;
  extern __shared__ __attribute__((aligned(1024))) uint8_t s_res[];
  const int Kp = (K + 31) & ~31;
  uint8_t* lc = s_res;
  float* lq = reinterpret_cast<float*>(s_res + (size_t)Kp * ROWB);

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, g = lane >> 4;
  const int b = blockIdx.y;
  const uint16_t* xb = x + (size_t)b * N * DP;
  const uint16_t* cb = cent + (size_t)b * K * DP;
  const float* qb = c_sq + (size_t)b * K;

  // This wave's first point tile is loaded before the table fill, so its
  // HBM round trip overlaps the fill's.  Points past N load point N-1
  // (their labels are not stored).
  const int ntiles = (N + 16 * PT - 1) / (16 * PT);
  int ts = blockIdx.x * W + wave;
  u32x4 xr[PT][DS2];
  auto load_points = [&](int tile) {
    const int n0 = min(tile, ntiles - 1) * 16 * PT;
#pragma unroll
    for (int p = 0; p < PT; ++p) {
      const int n = min(n0 + 16 * p + col, N - 1);
      const u32x4* src = reinterpret_cast<const u32x4*>(xb + (size_t)n * DP);
#pragma unroll
      for (int s = 0; s < DS2; ++s) xr[p][s] = src[4 * s + g];
    }
  };
  load_points(ts);

  // Table fill, CH 16-byte loads in flight per thread.  Row r keeps feature
  // segment v in slot v ^ swz(r), so a fragment read (16 consecutive rows)
  // touches 16 distinct bank groups; rows K..Kp-1 repeat row K-1 and get
  // the seed -inf, so they never win.
  {
    constexpr int CH = 8;
    const int total = Kp * SEGS;
    for (int i0 = 0; i0 < total; i0 += NTH * CH) {
      u32x4 v[CH];
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        const int i = min(i0 + j * NTH + tid, total - 1);
        const int r = i / SEGS, s = i % SEGS;
        v[j] = *reinterpret_cast<const u32x4*>(cb + (size_t)min(r, K - 1) * DP +
                                               s * 8);
      }
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        const int i = i0 + j * NTH + tid;
        if (i < total) {
          const int r = i / SEGS, s = i % SEGS;
          *reinterpret_cast<u32x4*>(lc + r * ROWB + ((s ^ swz<SEGS>(r)) * 16)) =
              v[j];
        }
      }
    }
    for (int k = tid; k < Kp; k += NTH) lq[k] = k < K ? -0.5f * qb[k] : -INFINITY;
  }
  __syncthreads();

  const int nblk = Kp >> 4;
  const int sw = swz<SEGS>(col);  // rows 16t + col share it
  auto frag = [&](int t, u32x4* a, f32x4& ci) {
    ci = *reinterpret_cast<const f32x4*>(lq + 16 * t + 4 * g);
    const uint8_t* arow = lc + (16 * t + col) * ROWB;
#pragma unroll
    for (int s = 0; s < DS2; ++s)
      a[s] = *reinterpret_cast<const u32x4*>(arow + (((4 * s + g) ^ sw) * 16));
  };

  // Point tiles of this batch row, strided over the row's waves; the next
  // tile's points are loaded once this one's are no longer needed.
  // Issue priority by progress, in halves of each tile: the arbiter
  // prefers older waves, so without it the first waves of a SIMD finish
  // early and the last run alone with nothing to hide their latency; with
  // priority falling as a wave advances, the ones behind catch up.
  const int stride = gridDim.x * W;
  const int mine = ts < ntiles ? (ntiles - ts + stride - 1) / stride : 1;
  for (int k = 0; ts < ntiles; ts += stride, ++k) {
    const int n0 = ts * 16 * PT;
    progress_prio(2 * k, 2 * mine);
    float best[PT];
    int bblk[PT];
#pragma unroll
    for (int p = 0; p < PT; ++p) {
      best[p] = -INFINITY;
      bblk[p] = 0;
    }
    // Two blocks per trip with ping-pong registers (no copies): block t's
    // MFMAs run while block t+1's fragments are read and block t-1 is
    // folded; the table has an even number of blocks (Kp % 32 == 0).  The
    // fold of the -inf seed before block 0 changes nothing, and the read
    // past the last block lands in the table's padding (resident_bytes) and
    // is never used: unclamped, the third read of a trip is the first one's
    // address plus a constant, so it costs no address arithmetic (measured
    // 1.5-2.5% faster at D = 32 and 64 than wrapping to block 0, the same
    // labels).  Eight tiles have no registers
    // for a second accumulator set: each block is folded after its own
    // MFMAs (the other waves of the SIMD cover the wait).
    u32x4 a0[DS2], a1[DS2];
    f32x4 c0, c1;
    f32x4 accA[PT], accB[PT];
#pragma unroll
    for (int p = 0; p < PT; ++p)
      accB[p] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    auto chain = [&](const u32x4* a, const f32x4& ci, f32x4* acc) {
#pragma unroll
      for (int s = 0; s < DS2; ++s) {
#pragma unroll
        for (int p = 0; p < PT; ++p)
          acc[p] = mfma16<DT>(a[s], xr[p][s], s == 0 ? ci : acc[p]);
      }
    };
    auto fold = [&](const f32x4* acc, int blk) {
#pragma unroll
      for (int p = 0; p < PT; ++p) fold_block(acc[p], best[p], bblk[p], blk);
    };
    auto hint = [&]() {
      if constexpr (FKC_SCHED_GROUPS && PT < 8) {
        __builtin_amdgcn_sched_group_barrier(0x100, DS2 + 1, 0);  // LDS reads
#pragma unroll
        for (int i = 0; i < DS2 * PT; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);  // VALU
        }
      }
    };
    frag(0, a0, c0);
    for (int t = 0; t < nblk; t += 2) {
      if (t == (nblk >> 2) * 2) progress_prio(2 * k + 1, 2 * mine);
      frag(t + 1, a1, c1);
      chain(a0, c0, accA);
      if constexpr (PT >= 8)
        fold(accA, 16 * t);
      else
        fold(accB, 16 * (t - 1));
      hint();
      frag(t + 2, a0, c0);
      chain(a1, c1, accB);
      if constexpr (PT >= 8)
        fold(accB, 16 * (t + 1));
      else
        fold(accA, 16 * t);
      hint();
    }
    if constexpr (PT < 8) fold(accB, 16 * (nblk - 1));

    // Settle each point as the staged kernel does (higher score, ties to
    // the lower candidate base; then the first of the four candidate rows
    // reaching the maximum of the re-scored diagonal), with the candidate
    // rows and seeds read from the LDS table.  base + r < Kp always.
    const int e = col & 3;
#pragma unroll
    for (int p = 0; p < PT; ++p) {
      float bv = best[p];
      int base = bblk[p] + 4 * g;
#pragma unroll
      for (int off = 16; off <= 32; off <<= 1) {
        const float ob = __shfl_xor(bv, off, 64);
        const int obase = __shfl_xor(base, off, 64);
        if (ob > bv || (ob == bv && obase < base)) {
          bv = ob;
          base = obase;
        }
      }
      float dv[4];
      const f32x4 seeds = *reinterpret_cast<const f32x4*>(lq + base);  // base % 4 == 0
      // Candidate rows from the table (their random rows cost LDS bank
      // conflicts, ~10 cycles per read at c4's shape, but reading them from
      // L2 instead, as the staged kernel does, measured 6% slower there).
      u32x4 ar[4][DS2];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kr = base + r;
        const uint8_t* crow = lc + kr * ROWB;
        const int ksw = swz<SEGS>(kr);
#pragma unroll
        for (int s = 0; s < DS2; ++s)
          ar[r][s] = *reinterpret_cast<const u32x4*>(crow + (((4 * s + g) ^ ksw) * 16));
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float seed = seeds[r];
        f32x4 acc = {seed, seed, seed, seed};
#pragma unroll
        for (int s = 0; s < DS2; ++s) acc = mfma16<DT>(ar[r][s], xr[p][s], acc);
        float d = acc[0];
        d = e == 1 ? acc[1] : d;
        d = e == 2 ? acc[2] : d;
        d = e == 3 ? acc[3] : d;
        dv[r] = d;
      }
      int rr = 0;
      float m = dv[0];
#pragma unroll
      for (int r = 1; r < 4; ++r) {
        if (dv[r] > m) {
          m = dv[r];
          rr = r;
        }
      }
      const int n = n0 + 16 * p + col;
      if (g == (col >> 2) && n < N) ids[(size_t)b * N + n] = base + rr;
    }
    if (ts + stride < ntiles) load_points(ts + stride);
  }
}

// Workgroups per batch row of a resident launch: one round of the chip
// (workgroups per CU set by the table's LDS), no more than the row's tiles
// need.
static int64_t resident_need(int pt, int w, int64_t N) {
  const int64_t tiles = (N + 16 * pt - 1) / (16 * pt);
  return (tiles + w - 1) / w;
}

static int resident_grid(int pt, int w, int64_t B, int64_t N) {
  const int64_t fill = std::max<int64_t>(1, device_shape().cus / B);
  return (int)std::max<int64_t>(1, std::min(resident_need(pt, w, N), fill));
}

template <int DT, int DS2, int PT, int W>
int launch_resident_t(const void* x, const void* c, const float* c_sq,
                      int32_t* ids, int64_t B, int64_t N, int64_t K,
                      const int32_t* ctrl, hipStream_t s, hipEvent_t ev0,
                      hipEvent_t ev1) {
  // Dynamic LDS above the default limit needs the kernel's attribute raised,
  // once per device (a bit per device id; the call is not a stream
  // operation, so it is also allowed while the stream is being captured).
  static std::atomic<uint64_t> raised{0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return fail(FKC_ERR_LAUNCH, "assign_resident: no current device");
  if (!(raised.load(std::memory_order_acquire) & (1ull << dev))) {
    const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&assign_resident_kernel<DT, DS2, PT, W>),
        hipFuncAttributeMaxDynamicSharedMemorySize,
        device_shape().lds_per_wg);
    if (attr != hipSuccess)
      return fail(FKC_ERR_LAUNCH, "assign_resident: LDS attribute: %s",
                  hipGetErrorString(attr));
    raised.fetch_or(1ull << dev, std::memory_order_acq_rel);
  }
  const int Kp = (int)((K + 31) & ~31);
  const size_t lds = (size_t)resident_bytes(DS2, Kp);
  dim3 grid((unsigned)resident_grid(PT, W, B, N), (unsigned)B);
  if (ev0 != nullptr)
    hipExtLaunchKernelGGL((assign_resident_kernel<DT, DS2, PT, W>), grid,
                          dim3(W * 64), lds, s, ev0, ev1, 0,
                          static_cast<const uint16_t*>(x),
                          static_cast<const uint16_t*>(c), c_sq, ids, (int)N,
                          (int)K, ctrl);
  else
    hipLaunchKernelGGL((assign_resident_kernel<DT, DS2, PT, W>), grid,
                       dim3(W * 64), lds, s,
                       static_cast<const uint16_t*>(x),
                       static_cast<const uint16_t*>(c), c_sq, ids, (int)N,
                       (int)K, ctrl);
  return check_launch("assign_resident");
}

// Centroid slicing of one launch: S slices of kspan rows (S = 1: none);
// psc / pidx hold B x S x N partial winners when S > 1.
struct Slices {
  int S = 1;
  int kspan = 0;
  float* psc = nullptr;
  int32_t* pidx = nullptr;
};

// ev0 / ev1 (both null or both set): events that the dispatch packets
// themselves stamp, ev0 at the start of the scoring kernel and ev1 at the
// end of the last kernel (no marker packets in the stream).
template <int DT, int DS2, int PT, bool PAD, bool EXACT, bool SAVE,
          bool WHOLE = false>
int launch_mfma_t(const void* x, const void* c, const float* c_sq,
                  int32_t* ids, int64_t B, int64_t N, int64_t K, int64_t D,
                  const int32_t* ctrl, const Slices& sl, hipStream_t s,
                  hipEvent_t ev0, hipEvent_t ev1) {
  constexpr int PTS_WG = 4 * PT * 16;
  const bool merge = sl.S > 1;
  dim3 grid((unsigned)((N + PTS_WG - 1) / PTS_WG), (unsigned)B,
            (unsigned)sl.S);
  const int kspan = merge ? sl.kspan : (int)K;
  if (ev0 != nullptr)
    hipExtLaunchKernelGGL((assign_mfma_kernel<DT, DS2, PT, PAD, EXACT, SAVE, WHOLE>), grid,
                          dim3(THREADS), 0, s, ev0, merge ? nullptr : ev1, 0,
                          static_cast<const uint16_t*>(x),
                          static_cast<const uint16_t*>(c), c_sq, ids, (int)N,
                          (int)K, (int)D, ctrl, kspan, sl.psc, sl.pidx);
  else
    hipLaunchKernelGGL((assign_mfma_kernel<DT, DS2, PT, PAD, EXACT, SAVE, WHOLE>), grid,
                       dim3(THREADS), 0, s, static_cast<const uint16_t*>(x),
                       static_cast<const uint16_t*>(c), c_sq, ids, (int)N,
                       (int)K, (int)D, ctrl, kspan, sl.psc, sl.pidx);
  if (int rc = check_launch("assign_mfma")) return rc;
  if (!merge) return FKC_OK;
  dim3 mgrid((unsigned)((N + 255) / 256), (unsigned)B);
  if (ev1 != nullptr)
    hipExtLaunchKernelGGL(assign_merge_kernel, mgrid, dim3(256), 0, s, nullptr,
                          ev1, 0, sl.psc, sl.pidx, ids, (int)N, sl.S, ctrl);
  else
    hipLaunchKernelGGL(assign_merge_kernel, mgrid, dim3(256), 0, s, sl.psc,
                       sl.pidx, ids, (int)N, sl.S, ctrl);
  return check_launch("assign_merge");
}

using MfmaLauncher = int (*)(const void*, const void*, const float*, int32_t*,
                             int64_t, int64_t, int64_t, int64_t,
                             const int32_t*, const Slices&, hipStream_t,
                             hipEvent_t, hipEvent_t);

template <int DT, int DS2, int PT>
constexpr MfmaLauncher entry(bool pad, bool exact, bool save, bool whole) {
  if constexpr (PT == 8) {
    // Direct stages and the re-score epilogue only (DS2 = 4, unpadded).
    if constexpr (DS2 == 4) {
      if (!pad && !exact && !save)
        return &launch_mfma_t<DT, DS2, PT, false, false, false>;
    }
    return nullptr;
  } else if constexpr (PT * DS2 * 4 <= 64) {
    if (save) {
      // Saved-score fold: four tiles at D = 64 or 97..128, unpadded only.
      if constexpr (PT == 4 && (DS2 == 4 || DS2 == 2)) {
        if (!pad && !exact) return &launch_mfma_t<DT, DS2, PT, false, false, true>;
      }
      return nullptr;
    }
    if constexpr (DS2 == 1 || DS2 == 2 || DS2 == 4 || DS2 == 8) {
      // One whole-table stage: exact index, unpadded, direct stages.
      if (whole && exact && !pad)
        return &launch_mfma_t<DT, DS2, PT, false, true, false, true>;
    }
    if (exact)
      return pad ? &launch_mfma_t<DT, DS2, PT, true, true, false>
                 : &launch_mfma_t<DT, DS2, PT, false, true, false>;
    return pad ? &launch_mfma_t<DT, DS2, PT, true, false, false>
               : &launch_mfma_t<DT, DS2, PT, false, false, false>;
  } else {
    return nullptr;
  }
}

// pt: 16-point tiles per wave (1, 2, 4, or 8 for unpadded D = 128 with the
// re-score epilogue).  The 1/2/4 variants keep the point registers
// (PT * DS2 * 4 VGPRs) at <= 64; the eight-tile one holds 128.
template <int DT, int DS2>
MfmaLauncher by_pt(int pt, bool pad, bool exact, bool save, bool whole) {
  switch (pt) {
    case 1: return entry<DT, DS2, 1>(pad, exact, save, whole);
    case 2: return entry<DT, DS2, 2>(pad, exact, save, whole);
    case 4: return entry<DT, DS2, 4>(pad, exact, save, whole);
    case 8: return entry<DT, DS2, 8>(pad, exact, save, whole);
    default: return nullptr;
  }
}

template <int DT>
MfmaLauncher mfma_launcher(int ds2, int pt, bool pad, bool exact, bool save,
                           bool whole) {
  switch (ds2) {
    case 1: return by_pt<DT, 1>(pt, pad, exact, save, whole);
    case 2: return by_pt<DT, 2>(pt, pad, exact, save, whole);
    case 3: return by_pt<DT, 3>(pt, pad, exact, save, whole);
    case 4: return by_pt<DT, 4>(pt, pad, exact, save, whole);
    case 5: return by_pt<DT, 5>(pt, pad, exact, save, whole);
    case 6: return by_pt<DT, 6>(pt, pad, exact, save, whole);
    case 7: return by_pt<DT, 7>(pt, pad, exact, save, whole);
    case 8: return by_pt<DT, 8>(pt, pad, exact, save, whole);
    case 9: return by_pt<DT, 9>(pt, pad, exact, save, whole);
    case 10: return by_pt<DT, 10>(pt, pad, exact, save, whole);
    case 11: return by_pt<DT, 11>(pt, pad, exact, save, whole);
    case 12: return by_pt<DT, 12>(pt, pad, exact, save, whole);
    case 13: return by_pt<DT, 13>(pt, pad, exact, save, whole);
    case 14: return by_pt<DT, 14>(pt, pad, exact, save, whole);
    case 15: return by_pt<DT, 15>(pt, pad, exact, save, whole);
    case 16: return by_pt<DT, 16>(pt, pad, exact, save, whole);
    default: return nullptr;
  }
}

}  // namespace

bool assign_uses_mfma(int dtype, int64_t D) {
  return (dtype == FKC_F16 || dtype == FKC_BF16) && D % 8 == 0 && D > 0 &&
         D <= 512 && !force_safe_assign();
}

// Workgroups an unsliced launch of pt tiles needs to fill the chip: 4 per
// CU in general; one per CU (one wave per SIMD) suffices for four tiles at
// D = 97..128, whose 16 MFMAs per centroid block keep a lone wave busy
// (measured on MI355X's 256 CUs at N = 131072, K = 2048 and N = 65536,
// K = 8192: four tiles on 512 / 256 workgroups beat two tiles on 1024 / 512
// by 3% / 5%); eight tiles run 2 workgroups per CU and need two rounds of
// them.
static int64_t fill_wgs(int pt, int ds2, bool exact) {
  const int64_t cus = device_shape().cus;
  return (!exact && pt == 4 && ds2 == 4) ? cus : 4 * cus;
}

static int64_t grid_wgs(int pt, int64_t B, int64_t N) {
  return B * ((N + 64 * pt - 1) / (64 * pt));
}

static bool pt8_ok(int ds2, bool pad, bool exact) {
  return ds2 == 4 && !pad && !exact;
}

// Tiles per wave for an unsliced launch: the largest of 8 (unpadded
// D = 128, re-score epilogue only), 4, 2, 1 (bounded by the 64-VGPR point
// budget) whose grid fills the chip (fill_wgs); fewer, fatter workgroups
// reuse each LDS centroid stage more, but grids that leave CUs idle hide
// latency badly (measured at the c2..c5 shapes; eight tiles at D = 64 ran
// slower than four).  From K = 8192 one full round of eight-tile
// workgroups (2 per CU) is enough: their longer loop amortizes the
// prologue and re-score (fp16, N = 256 x four-tile workgroups, same box,
// interleaved: 1024 / 1280 / 1536 workgroups' worth of points at
// K = 8192 -3.3% / -0.4% / -1.3%, at K = 16384 -6.1% / -4.2% / -4.0%;
// at K = 4096 one or one and a half rounds lose, +8% to +12%).
// FKC_NTILES overrides where the variant exists.
static int choose_pt(int ds2, bool pad, bool exact, int64_t B, int64_t N,
                     int64_t K) {
  const int o = ntiles_override();
  if (o == 8 && pt8_ok(ds2, pad, exact)) return o;
  if (o != 0 && o != 8 && o * ds2 * 4 <= 64) return o;
  for (int pt = 8; pt > 1; pt >>= 1) {
    if (pt == 8 ? !pt8_ok(ds2, pad, exact) : pt * ds2 * 4 > 64) continue;
    if (grid_wgs(pt, B, N) >= fill_wgs(pt, ds2, exact)) return pt;
    if (pt == 8 && K >= 8192 && grid_wgs(8, B, N) >= 2 * device_shape().cus)
      return 8;
  }
  return 1;
}

struct Plan {
  int ds2, pt, S, kspan;
  bool pad, exact, save;
  bool whole = false;  // exact index, the table in one direct stage
  bool resident = false;  // assign_resident_kernel (pt: its tiles per wave)
};

// The saved-score fold keeps the best block's four scores per lane, so the
// winner needs no re-score: the re-score reads four full candidate rows per
// point (512 B at D = 64, bf16), which at the end of a round of workgroups
// is all CU-L1 traffic with the matrix cores idle.  Four tiles, unpadded.
// At D = 97..128 it runs two workgroups per CU against the re-score's
// three, so besides skipping the re-score it changes how whole the rounds
// of workgroups are: a round that is a fraction of the slots ends with
// CUs running one workgroup.  It is taken where K (per slice) <= 2048 at
// any grid, and up to K = 8191 where its rounds are whole enough
// (round_fill below) to beat the re-score's by 0.15; at K >= 8192 only on
// grids of at most two workgroups per CU.  Same-box fp16 assign times over
// grids of 256..1536 workgroups and K = 1024..8192 (N = 256 x workgroups),
// save against re-score: K = 1024 -24% to -31% from 640 workgroups on,
// K = 2048 -2% to -17% (c3's 512: +1%), K = 3072 / 4096 at 896 and 1024
// workgroups -9% / -6% and -5% / -2%, at 640, 768, 1280, 1536 +3% to +9%;
// K = 8192 at 1024 +3%.  At D = 64 it costs a wave per SIMD (163 VGPRs,
// three waves) and four selects per 16-centroid block, which pays for K
// (per slice) <= 1024 (same-box assign times against the re-score, bf16:
// (4, 100000, 600) -25%, (1, 262144, 1024) -9.6%, (8, 65536, 1024) -2.4% to
// -6.7%; but (8, 65536, 2048) +8.3%, (1, 524288, 2048) +7.6%, K = 4096 /
// 8192 +14 / +15%).  FKC_SAVE=0/1 forces it off / on where it exists.
static double round_fill(int64_t wgs, int64_t slots) {
  const int64_t rounds = (wgs + slots - 1) / slots;
  return (double)wgs / (double)(rounds * slots);
}

static bool use_save(const Plan& p, int64_t wgs) {
  if (p.pt != 4 || (p.ds2 != 4 && p.ds2 != 2) || p.pad || p.exact) return false;
  const int o = save_override();
  if (o >= 0) return o == 1;
  if (p.ds2 == 2) return p.kspan <= 1024;
  const int64_t cus = device_shape().cus;
  if (p.kspan <= 2048) return true;
  if (p.kspan >= 8192) return wgs <= 2 * cus;
  return round_fill(wgs, 2 * cus) >= round_fill(wgs, 3 * cus) + 0.15;
}

// Tiles per wave of the resident kernel.
static int resident_pt(int ds2) { return ds2 == 1 ? 8 : 4; }

// The centroid-resident kernel: unpadded D = 32 or 64 whose centroid table
// fits one workgroup's LDS.  Taken where its grid gives every CU a
// workgroup and K is past the exact-index cutoff (measured: fewer
// workgroups than CUs leave the table fill and the first point loads
// unhidden, and at small K the staged kernel's exact fold is as fast).
// FKC_RESIDENT=0/1 forces it off / on where the table fits.
static bool use_resident(const Plan& p, int64_t B, int64_t N, int64_t K) {
  if (p.pad || (p.ds2 != 1 && p.ds2 != 2)) return false;
  const int64_t Kp = (K + 31) & ~int64_t{31};
  const DeviceShape dev = device_shape();
  if (Kp > 65536 || resident_bytes(p.ds2, (int)Kp) > dev.lds_per_wg)
    return false;
  const int o = resident_override();
  if (o >= 0) return o == 1;
  const int pt = resident_pt(p.ds2);
  return K > FKC_EXACT_MAX_K_NARROW &&
         B * resident_need(pt, kResidentWaves, N) >= dev.cus;
}

// Launch plan.  K is sliced only when no unsliced grid fills the chip (few
// points, many centroids): the most tiles the point budget allows (four up
// to D = 128) then run on S slices of kspan rows
// (a multiple of 128, at least FKC_SLICE_MIN_ROWS) scored by separate
// workgroups, and a small kernel merges them.  Each slice re-reads its
// points and ends with its own re-score, so short slices lose: at
// N = 131072, K = 2048, D = 128 four slices of 512 rows took 0.124 ms
// against 0.073 ms unsliced; at N = 80000, K = 70000, D = 16 four slices
// took 0.376 ms against 0.756 ms, and at N = 8192, K = 65536, D = 128
// eight slices 0.150 ms against 0.531 ms.  At D = 97..128 the slices fill
// one round of resident workgroups (below).  FKC_KSPLIT forces S.
static Plan plan_assign(int64_t B, int64_t N, int64_t K, int64_t D,
                        bool can_slice) {
  Plan p;
  p.ds2 = (int)((D + 31) / 32);
  p.pad = D != 32 * p.ds2;
  // Re-scoring the winning block costs about one 16-centroid block per point
  // tile and one round trip for the candidate rows (all of a tile's loads
  // issued together); below this K the exact in-loop index is cheaper.  The
  // exact fold costs ~13 vector instructions per four scores against ~5,
  // which at D <= 64 (two MFMAs per block) makes it vector-ALU-bound: with
  // the batched re-score the block fold wins from K = 513 at every width
  // (same labels; (8, 65536, 1024, 64) bf16 0.0884 -> 0.0851 ms,
  // (1, 262144, 768, 32) 0.0288 -> 0.0238, (4, 100000, 1000, 48) 0.0752 ->
  // 0.0695).
  p.exact = K <= FKC_EXACT_MAX_K || (p.ds2 <= 2 && K <= FKC_EXACT_MAX_K_NARROW);
  p.pt = choose_pt(p.ds2, p.pad, p.exact, B, N, K);
  p.S = 1;
  p.kspan = (int)K;
  if (use_resident(p, B, N, K)) {
    p.resident = true;
    p.exact = false;
    p.save = false;
    p.pt = resident_pt(p.ds2);
    return p;
  }
  p.save = use_save(p, grid_wgs(p.pt, B, N));
  // One whole-table stage (64 KB at D = 128) where the table fits it and
  // the grid is one round of two workgroups per CU (the stage's LDS allows
  // two): one load round trip and one barrier instead of one per 64-row
  // stage.
  p.whole = FKC_WHOLE_STAGE && FKC_USE_DMA && p.exact && !p.pad &&
            (p.ds2 == 1 || p.ds2 == 2 || p.ds2 == 4 || p.ds2 == 8) &&
            K <= (p.ds2 <= 4 ? 256 : 128) &&
            grid_wgs(p.pt, B, N) <= 2 * device_shape().cus;
  if (!can_slice || p.exact) return p;
  // Four tiles, not eight: on sliced-size grids four tiles on ~256
  // workgroups beat eight on 512 (N = 8192, K = 65536: 0.150 vs 0.166 ms;
  // N = 16384, K = 32768: 0.142 vs 0.156 ms).
  int pt = p.pt;
  if (ntiles_override() == 0) pt = p.ds2 <= 4 ? 4 : p.ds2 <= 8 ? 2 : 1;
  const int64_t tiles = grid_wgs(pt, B, N);
  int64_t S = ksplit_override();
  if (S == 0 && pt == 4 && p.ds2 == 4) {
    // D = 97..128: as many slices as fit one round of the 167-VGPR
    // variant's resident workgroups (3 per CU, 768 on MI355X).  One round,
    // not two: at N = 65536, K = 8192 three slices took 0.117 ms, four
    // 0.122, none 0.121; at N = 32768, K = 16384 six 0.123, three 0.138,
    // none 0.220; at N = 131072, K = 4096 two slices (two rounds) lost 6%.
    // Where whole slices of at most 4096 rows also fill one round of the
    // kept-score variant's workgroups (2 per CU) as fully, that round runs
    // with no re-score (same-box assign times, kept scores on 2 x CUs /
    // tiles slices against the re-score on 3 x CUs / tiles: N = 65536,
    // K = 8192 0.112 vs 0.117 ms; N = 32768, K = 16384 0.112 vs 0.119;
    // N = 16384, K = 32768 0.113 vs 0.122; at 8192-row slices it lost,
    // 0.215 vs 0.209, and at N = 49152 (a three-quarter round) 0.096 vs
    // 0.088).
    const int64_t cus = device_shape().cus;
    const int64_t s3 = std::min<int64_t>(3 * cus / tiles, K / FKC_SLICE_MIN_ROWS);
    const int64_t s2 = std::min<int64_t>(2 * cus / tiles, K / FKC_SLICE_MIN_ROWS);
    S = s3;
    if (s2 >= 2) {
      const int64_t span2 = ((K + s2 - 1) / s2 + 127) / 128 * 128;
      if (span2 <= 4096 &&
          round_fill(tiles * s2, 2 * cus) >=
              round_fill(tiles * std::max<int64_t>(s3, 1), 3 * cus))
        S = s2;
    }
    if (S <= 1) return p;
  } else if (S == 0) {
    const int64_t want = fill_wgs(pt, p.ds2, p.exact);
    if (tiles >= want) return p;
    S = 1;
    while (tiles * S < want && K / (2 * S) >= FKC_SLICE_MIN_ROWS) S *= 2;
    // Slices that still leave the chip short only pay off when the unsliced
    // grid is short too.
    if (tiles * S < want &&
        grid_wgs(p.pt, B, N) >= fill_wgs(p.pt, p.ds2, p.exact))
      return p;
  }
  const int64_t span = ((K + S - 1) / S + 127) / 128 * 128;
  S = (K + span - 1) / span;
  if (S <= 1) return p;
  p.pt = pt;
  p.S = (int)S;
  p.kspan = (int)span;
  p.save = use_save(p, tiles * S);
  return p;
}

static size_t slice_bytes(const Plan& p, int64_t B, int64_t N, Slices* sl,
                          void* ws) {
  if (p.S <= 1) return 0;
  Carve c(ws);
  float* psc = c.take<float>((size_t)B * p.S * N);
  int32_t* pidx = c.take<int32_t>((size_t)B * p.S * N);
  if (sl) {
    sl->S = p.S;
    sl->kspan = p.kspan;
    sl->psc = psc;
    sl->pidx = pidx;
  }
  return c.used;
}

size_t assign_workspace_bytes(int64_t B, int64_t N, int64_t K, int64_t D,
                              int dtype) {
  if (!assign_uses_mfma(dtype, D) || B * N == 0 || K < 1) return 0;
  return slice_bytes(plan_assign(B, N, K, D, true), B, N, nullptr, nullptr);
}

int launch_assign_mfma(const void* x, const void* c, const float* c_sq,
                       int32_t* ids, int64_t B, int64_t N, int64_t K,
                       int64_t D, int dtype, const int32_t* ctrl,
                       hipStream_t s, hipEvent_t ev0, hipEvent_t ev1,
                       void* ws, size_t ws_bytes) {
  const Plan p = plan_assign(B, N, K, D, ws != nullptr);
  if (p.resident) {
    using RL = int (*)(const void*, const void*, const float*, int32_t*,
                       int64_t, int64_t, int64_t, const int32_t*, hipStream_t,
                       hipEvent_t, hipEvent_t);
    constexpr int W = kResidentWaves;
    const bool f16 = dtype == FKC_F16;
    RL fn = p.ds2 == 1 ? (f16 ? &launch_resident_t<FKC_F16, 1, 8, W>
                              : &launch_resident_t<FKC_BF16, 1, 8, W>)
                       : (f16 ? &launch_resident_t<FKC_F16, 2, 4, W>
                              : &launch_resident_t<FKC_BF16, 2, 4, W>);
    return fn(x, c, c_sq, ids, B, N, K, ctrl, s, ev0, ev1);
  }
  Slices sl;
  const size_t need = slice_bytes(p, B, N, &sl, ws);
  if (need > ws_bytes)
    return fail(FKC_ERR_WORKSPACE, "assign: workspace %zu < %zu bytes",
                ws_bytes, need);
  MfmaLauncher fn =
      dtype == FKC_F16
          ? mfma_launcher<FKC_F16>(p.ds2, p.pt, p.pad, p.exact, p.save, p.whole)
          : mfma_launcher<FKC_BF16>(p.ds2, p.pt, p.pad, p.exact, p.save, p.whole);
  if (!fn)
    return fail(FKC_ERR_UNSUPPORTED, "assign: no MFMA variant for D=%lld",
                (long long)D);
  return fn(x, c, c_sq, ids, B, N, K, D, ctrl, sl, s, ev0, ev1);
}

}  // namespace fkc
