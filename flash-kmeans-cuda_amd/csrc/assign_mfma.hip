// Fused distance + argmin on gfx950 matrix cores (fp16 / bf16 inputs).
//
// What it computes (same ranking as the reference's raw-distance MMA route,
// flash_kmeans_cuda/csrc/assign/assign_sm80.cu:437-441 with RAW_DIST=true at
// :687): for every point n of batch b,
//     ids[b,n] = argmax_k ( <x_n, c_k> - c_sq[k]/2 )
//              = argmin_k ( c_sq[k] - 2 <x_n, c_k> ),
// the lowest k winning exact ties (assign_common.cuh:20-28,
// assign_sm80.cu:594-611).  x_sq is row-constant for the argmin and is not
// read.  Products are exact in fp32 and accumulate in fp32
// (the reference accumulates fp16 inputs in fp16, assign_sm80.cu:81-118).
//
// Mapping onto v_mfma_f32_32x32x16_{f16,bf16} (D = A*B + C, 32x32 tiles):
//   A (rows)    = 32 centroids  x 16 features, streamed through LDS;
//   B (columns) = 16 features x 32 points, held in VGPRs for the whole
//                 K loop (each lane owns one point's 8-feature slices);
//   C           = -c_sq/2 of the 32 centroids, so the accumulator leaves the
//                 matrix core already holding the score to maximise;
//                 centroids past K get -inf and can never win.
// Lane l holds column (point) l%32 and rows 8g + 4(l/32) + r (g,r in 0..3),
// i.e. 16 scores of one point against centroids in increasing order.  Per
// tile a lane takes the max of its 16 scores (max3 tree); only when that max
// beats the lane's running best does it search for the first matching slot,
// so the index bookkeeping costs almost nothing once the best has settled.
// Lanes l and l+32 (same point, interleaved centroid rows) merge at the end
// with the lowest-index tie rule.
//
// Workgroup: 4 waves x PT point tiles x 32 points.  Centroids move through
// LDS in stages of 64 rows (row stride D+8 halves: the 16-byte pad spreads
// the 32 rows a ds_read_b128 touches over all 64 banks), double-buffered
// with one barrier per stage; the next stage's global loads are in flight
// while the matrix cores work on the current one.
#include "device_util.hpp"
#include "fkc_internal.hpp"

#include <math.h>

namespace fkc {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int KC = 64;        // centroid rows per LDS stage
constexpr int THREADS = 256;  // 4 waves

template <int DT>
__device__ inline f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c);

template <>
__device__ inline f32x16 mfma32<FKC_F16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(
      __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <>
__device__ inline f32x16 mfma32<FKC_BF16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
      __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
      0);
}

// Fold one tile's 16 scores into the lane's running (best, index).
// kt = global index of the lane's slot 0; slot v maps to kt + 8(v/4) + v%4.
__device__ inline void fold_tile(const f32x16& acc, float& best, int& bidx,
                                 int kt) {
  float m0 = fmaxf(fmaxf(acc[0], acc[1]), acc[2]);
  float m1 = fmaxf(fmaxf(acc[3], acc[4]), acc[5]);
  float m2 = fmaxf(fmaxf(acc[6], acc[7]), acc[8]);
  float m3 = fmaxf(fmaxf(acc[9], acc[10]), acc[11]);
  float m4 = fmaxf(fmaxf(acc[12], acc[13]), acc[14]);
  float m5 = fmaxf(fmaxf(m0, m1), m2);
  float m6 = fmaxf(fmaxf(m3, m4), acc[15]);
  float m = fmaxf(m5, m6);
  if (m > best) {  // strict: an equal score seen later has a larger index
    int sel = 15;
#pragma unroll
    for (int v = 14; v >= 0; --v) sel = (acc[v] == m) ? v : sel;
    best = m;
    bidx = kt + 8 * (sel >> 2) + (sel & 3);
  }
}

template <int DT, int DS, int PT>
__global__ void __launch_bounds__(THREADS, (PT * DS <= 16) ? 2 : 1)
assign_mfma_kernel(const uint16_t* __restrict__ x,
                   const uint16_t* __restrict__ cent,
                   const float* __restrict__ c_sq, int32_t* __restrict__ ids,
                   int N, int K, const int32_t* __restrict__ ctrl) {
  if (loop_done(ctrl)) return;
  constexpr int D = DS * 16;
  constexpr int ROW = D + 8;  // LDS row stride in 16-bit elements
  constexpr int SEGS = DS * 2;  // 16-byte segments per centroid row
  constexpr int PIECES = KC * SEGS;
  constexpr int PPT = (PIECES + THREADS - 1) / THREADS;
  constexpr int PTS_WAVE = PT * 32;
  constexpr int PTS_WG = 4 * PTS_WAVE;

  __shared__ __attribute__((aligned(16))) uint16_t lds_c[2][KC * ROW];
  __shared__ __attribute__((aligned(16))) float lds_q[2][KC];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, h = lane >> 5;
  const int b = blockIdx.y;
  const uint16_t* xb = x + (size_t)b * N * D;
  const uint16_t* cb = cent + (size_t)b * K * D;
  const float* qb = c_sq + (size_t)b * K;
  const int n0 = blockIdx.x * PTS_WG + wave * PTS_WAVE;

  // B operand: this lane's point, features 16s + 8h .. +7 for every step s.
  u32x4 xr[PT][DS];
#pragma unroll
  for (int p = 0; p < PT; ++p) {
    const int n = n0 + 32 * p + col;
    if (n < N) {
      const u32x4* src = reinterpret_cast<const u32x4*>(xb + (size_t)n * D) + h;
#pragma unroll
      for (int s = 0; s < DS; ++s) xr[p][s] = src[2 * s];
    } else {
#pragma unroll
      for (int s = 0; s < DS; ++s) xr[p][s] = u32x4{0u, 0u, 0u, 0u};
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
        const int k = kb + r;
        pf[j] = (k < K)
                    ? reinterpret_cast<const u32x4*>(cb + (size_t)k * D)[sg]
                    : u32x4{0u, 0u, 0u, 0u};
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
    for (int t = 0; t < KC / 32; ++t) {
      f32x16 cinit;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 q =
            *reinterpret_cast<const float4*>(lq + 32 * t + 8 * g + 4 * h);
        cinit[4 * g + 0] = q.x;
        cinit[4 * g + 1] = q.y;
        cinit[4 * g + 2] = q.z;
        cinit[4 * g + 3] = q.w;
      }
      f32x16 acc[PT];
#pragma unroll
      for (int p = 0; p < PT; ++p) acc[p] = cinit;
      const u32x4* arow =
          reinterpret_cast<const u32x4*>(lc + (32 * t + col) * ROW) + h;
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        const u32x4 a = arow[2 * s];
#pragma unroll
        for (int p = 0; p < PT; ++p) acc[p] = mfma32<DT>(a, xr[p][s], acc[p]);
      }
      const int kt = chunk * KC + 32 * t + 4 * h;
#pragma unroll
      for (int p = 0; p < PT; ++p) fold_tile(acc[p], best[p], bidx[p], kt);
    }
    if (chunk + 1 < nchunks) lstore(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int p = 0; p < PT; ++p) {
    const float ob = __shfl_xor(best[p], 32, 64);
    const int oi = __shfl_xor(bidx[p], 32, 64);
    if (ob > best[p] || (ob == best[p] && oi < bidx[p])) {
      best[p] = ob;
      bidx[p] = oi;
    }
    const int n = n0 + 32 * p + col;
    if (h == 0 && n < N) ids[(size_t)b * N + n] = bidx[p];
  }
}

template <int DT, int DS, int PT>
int launch_mfma_t(const void* x, const void* c, const float* c_sq,
                  int32_t* ids, int64_t B, int64_t N, int64_t K,
                  const int32_t* ctrl, hipStream_t s) {
  constexpr int PTS_WG = 4 * PT * 32;
  dim3 grid((unsigned)((N + PTS_WG - 1) / PTS_WG), (unsigned)B);
  hipLaunchKernelGGL((assign_mfma_kernel<DT, DS, PT>), grid, dim3(THREADS), 0,
                     s, static_cast<const uint16_t*>(x),
                     static_cast<const uint16_t*>(c), c_sq, ids, (int)N,
                     (int)K, ctrl);
  return check_launch("assign_mfma");
}

using MfmaLauncher = int (*)(const void*, const void*, const float*, int32_t*,
                             int64_t, int64_t, int64_t, const int32_t*,
                             hipStream_t);

// Default point tiles per wave: keep the point registers at <= 64 VGPRs
// (4 tiles for D <= 64, 2 for D <= 128, 1 above) so two waves share a SIMD.
constexpr int default_pt(int ds) { return ds <= 4 ? 4 : (ds <= 8 ? 2 : 1); }

template <int DT, int DS>
MfmaLauncher by_pt(int pt) {
  // FKC_NTILES variants are built for D = 64 and D = 128 only.
  if constexpr (DS == 4 || DS == 8) {
    if (pt == 1) return &launch_mfma_t<DT, DS, 1>;
    if (pt == 2) return &launch_mfma_t<DT, DS, 2>;
    if (pt == 4) return &launch_mfma_t<DT, DS, 4>;
  }
  (void)pt;
  return &launch_mfma_t<DT, DS, default_pt(DS)>;
}

template <int DT>
MfmaLauncher mfma_launcher(int ds, int pt) {
  switch (ds) {
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
  return (dtype == FKC_F16 || dtype == FKC_BF16) && D % 16 == 0 && D > 0 &&
         D <= 256 && !force_safe_assign();
}

int launch_assign_mfma(const void* x, const void* c, const float* c_sq,
                       int32_t* ids, int64_t B, int64_t N, int64_t K,
                       int64_t D, int dtype, const int32_t* ctrl,
                       hipStream_t s) {
  const int ds = (int)(D / 16);
  const int pt = ntiles_override();  // 0 = default for this D
  MfmaLauncher fn = dtype == FKC_F16 ? mfma_launcher<FKC_F16>(ds, pt)
                                     : mfma_launcher<FKC_BF16>(ds, pt);
  if (!fn) return fail(FKC_ERR_UNSUPPORTED, "assign: no MFMA variant for D=%lld",
                       (long long)D);
  return fn(x, c, c_sq, ids, B, N, K, ctrl, s);
}

}  // namespace fkc
