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
// of one point against consecutive centroids.  A lane keeps a running
// (best, index); a tile's max is compared once, and only when it beats the
// best does the lane look for the first matching slot.  The four lanes that
// share a point (l, l+16, l+32, l+48) merge at the end with the lowest-index
// rule.  Feature widths that are not a multiple of 32 are zero-padded in
// registers and LDS (zeros add nothing to a dot product).
//
// Workgroup: 4 waves x PT point tiles x 16 points (PT chosen per grid size).  Centroids pass through LDS
// in stages of 64 rows (row stride DP+8 halves: the 16-byte pad spreads the
// rows a ds_read_b128 touches over distinct banks), double-buffered with one
// barrier per stage; the next stage's global loads are in flight while the
// matrix cores work on the current one.  Centroid rows past K re-read row
// K-1 instead of branching (their scores are masked).
#include "device_util.hpp"
#include "fkc_internal.hpp"

#include <math.h>

namespace fkc {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int KC = 64;        // centroid rows per LDS stage
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

// Fold four scores (centroids kt..kt+3) into the running (best, index).
__device__ inline void fold4(const f32x4& acc, float& best, int& bidx,
                             int kt) {
  const float m = fmaxf(fmaxf(fmaxf(acc[0], acc[1]), acc[2]), acc[3]);
  if (m > best) {  // strict: an equal score seen later has a larger index
    const int sel =
        acc[0] == m ? 0 : (acc[1] == m ? 1 : (acc[2] == m ? 2 : 3));
    best = m;
    bidx = kt + sel;
  }
}

// DS2: 32-feature steps (padded width DP = 32*DS2 >= D); PT: 16-point tiles
// per wave.  D % 8 == 0 so every 8-feature segment is a 16-byte load.
template <int DT, int DS2, int PT>
__global__ void __launch_bounds__(THREADS, (PT * DS2 <= 16) ? 2 : 1)
assign_mfma_kernel(const uint16_t* __restrict__ x,
                   const uint16_t* __restrict__ cent,
                   const float* __restrict__ c_sq, int32_t* __restrict__ ids,
                   int N, int K, int D, const int32_t* __restrict__ ctrl) {
  if (loop_done(ctrl)) return;
  constexpr int DP = DS2 * 32;
  constexpr int ROW = DP + 8;       // LDS row stride in 16-bit elements
  constexpr int SEGS = DP / 8;      // 16-byte segments per padded row
  constexpr int PIECES = KC * SEGS;
  constexpr int PPT = (PIECES + THREADS - 1) / THREADS;
  constexpr int PTS_WAVE = PT * 16;
  constexpr int PTS_WG = 4 * PTS_WAVE;
  constexpr int NT = KC / 16;

  __shared__ __attribute__((aligned(16))) uint16_t lds_c[2][KC * ROW];
  __shared__ __attribute__((aligned(16))) float lds_q[2][KC];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, g = lane >> 4;
  const int b = blockIdx.y;
  const int dsegs = D / 8;          // real segments per row
  const bool padded = dsegs != SEGS;
  const uint16_t* xb = x + (size_t)b * N * D;
  const uint16_t* cb = cent + (size_t)b * K * D;
  const float* qb = c_sq + (size_t)b * K;
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
      xr[p][s] = (!padded || seg < dsegs) ? src[seg] : u32x4{0u, 0u, 0u, 0u};
    }
  }

  float best[PT];
  int bidx[PT];
#pragma unroll
  for (int p = 0; p < PT; ++p) {
    best[p] = -INFINITY;
    bidx[p] = 0;
  }

  u32x4 pf[PPT];
  float pq = 0.f;
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
    if (tid < KC) {
      const int k = kb + tid;
      pq = (k < K) ? -0.5f * qb[k] : -INFINITY;
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int i = tid + j * THREADS;
      if (PIECES % THREADS == 0 || i < PIECES) {
        const int r = i / SEGS, sg = i % SEGS;
        *reinterpret_cast<u32x4*>(&lds_c[buf][r * ROW + sg * 8]) = pf[j];
      }
    }
    if (tid < KC) lds_q[buf][tid] = pq;
  };

  gload(0);
  lstore(0);
  __syncthreads();

  for (int chunk = 0; chunk < nchunks; ++chunk) {
    const int buf = chunk & 1;
    if (chunk + 1 < nchunks) gload(chunk + 1);
    const uint16_t* lc = lds_c[buf];
    const float* lq = lds_q[buf];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const f32x4 cinit = *reinterpret_cast<const f32x4*>(lq + 16 * t + 4 * g);
      const u32x4* arow =
          reinterpret_cast<const u32x4*>(lc + (16 * t + col) * ROW) + g;
      u32x4 a[DS2];
#pragma unroll
      for (int s = 0; s < DS2; ++s) a[s] = arow[4 * s];
      f32x4 acc[PT];
#pragma unroll
      for (int s = 0; s < DS2; ++s) {
#pragma unroll
        for (int p = 0; p < PT; ++p)
          acc[p] = mfma16<DT>(a[s], xr[p][s], s == 0 ? cinit : acc[p]);
      }
      const int kt = chunk * KC + 16 * t + 4 * g;
#pragma unroll
      for (int p = 0; p < PT; ++p) fold4(acc[p], best[p], bidx[p], kt);
    }
    if (chunk + 1 < nchunks) lstore(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int p = 0; p < PT; ++p) {
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1) {
      const float ob = __shfl_xor(best[p], off, 64);
      const int oi = __shfl_xor(bidx[p], off, 64);
      if (ob > best[p] || (ob == best[p] && oi < bidx[p])) {
        best[p] = ob;
        bidx[p] = oi;
      }
    }
    const int n = n0 + 16 * p + col;
    if (g == 0 && n < N) ids[(size_t)b * N + n] = bidx[p];
  }
}

template <int DT, int DS2, int PT>
int launch_mfma_t(const void* x, const void* c, const float* c_sq,
                  int32_t* ids, int64_t B, int64_t N, int64_t K, int64_t D,
                  const int32_t* ctrl, hipStream_t s) {
  constexpr int PTS_WG = 4 * PT * 16;
  dim3 grid((unsigned)((N + PTS_WG - 1) / PTS_WG), (unsigned)B);
  hipLaunchKernelGGL((assign_mfma_kernel<DT, DS2, PT>), grid, dim3(THREADS),
                     0, s, static_cast<const uint16_t*>(x),
                     static_cast<const uint16_t*>(c), c_sq, ids, (int)N,
                     (int)K, (int)D, ctrl);
  return check_launch("assign_mfma");
}

using MfmaLauncher = int (*)(const void*, const void*, const float*, int32_t*,
                             int64_t, int64_t, int64_t, int64_t,
                             const int32_t*, hipStream_t);

template <int DT, int DS2, int PT>
constexpr MfmaLauncher entry() {
  if constexpr (PT * DS2 * 4 <= 64 || (PT == 8 && (DS2 == 2 || DS2 == 4)))
    return &launch_mfma_t<DT, DS2, PT>;
  else
    return nullptr;
}

// pt: 16-point tiles per wave (1, 2, 4, or 8 for D = 64 / 128 only).
// Variants keep the point registers (PT * DS2 * 4 VGPRs) at <= 64.
template <int DT, int DS2>
MfmaLauncher by_pt(int pt) {
  switch (pt) {
    case 1: return entry<DT, DS2, 1>();
    case 2: return entry<DT, DS2, 2>();
    case 4: return entry<DT, DS2, 4>();
    case 8: return entry<DT, DS2, 8>();
    default: return nullptr;
  }
}

template <int DT>
MfmaLauncher mfma_launcher(int ds2, int pt) {
  switch (ds2) {
    case 1: return by_pt<DT, 1>(pt);
    case 2: return by_pt<DT, 2>(pt);
    case 3: return by_pt<DT, 3>(pt);
    case 4: return by_pt<DT, 4>(pt);
    case 5: return by_pt<DT, 5>(pt);
    case 6: return by_pt<DT, 6>(pt);
    case 7: return by_pt<DT, 7>(pt);
    case 8: return by_pt<DT, 8>(pt);
    case 9: return by_pt<DT, 9>(pt);
    case 10: return by_pt<DT, 10>(pt);
    case 11: return by_pt<DT, 11>(pt);
    case 12: return by_pt<DT, 12>(pt);
    case 13: return by_pt<DT, 13>(pt);
    case 14: return by_pt<DT, 14>(pt);
    case 15: return by_pt<DT, 15>(pt);
    case 16: return by_pt<DT, 16>(pt);
    default: return nullptr;
  }
}

}  // namespace

bool assign_uses_mfma(int dtype, int64_t D) {
  return (dtype == FKC_F16 || dtype == FKC_BF16) && D % 8 == 0 && D > 0 &&
         D <= 512 && !force_safe_assign();
}

// Tiles per wave: the largest of 4, 2, 1 (bounded by the 64-VGPR point
// budget) whose grid still has >= 1024 workgroups (4 per CU on 256 CUs);
// fewer, fatter workgroups reuse each LDS centroid stage more, but small
// grids leave CUs idle and hide latency badly (measured at the c2..c5
// shapes).  FKC_NTILES overrides.
static int choose_pt(int ds2, int64_t B, int64_t N) {
  const int o = ntiles_override();
  if (o != 0 && (o * ds2 * 4 <= 64 || (o == 8 && (ds2 == 2 || ds2 == 4))))
    return o;
  for (int pt = 4; pt > 1; pt >>= 1) {
    if (pt * ds2 * 4 > 64) continue;
    const int64_t wgs = B * ((N + 64 * pt - 1) / (64 * pt));
    if (wgs >= 1024) return pt;
  }
  return 1;
}

int launch_assign_mfma(const void* x, const void* c, const float* c_sq,
                       int32_t* ids, int64_t B, int64_t N, int64_t K,
                       int64_t D, int dtype, const int32_t* ctrl,
                       hipStream_t s) {
  const int ds2 = (int)((D + 31) / 32);
  const int pt = choose_pt(ds2, B, N);
  MfmaLauncher fn = dtype == FKC_F16 ? mfma_launcher<FKC_F16>(ds2, pt)
                                     : mfma_launcher<FKC_BF16>(ds2, pt);
  if (!fn)
    return fail(FKC_ERR_UNSUPPORTED, "assign: no MFMA variant for D=%lld",
                (long long)D);
  return fn(x, c, c_sq, ids, B, N, K, D, ctrl, s);
}

}  // namespace fkc
