// fp32 VALU assignment (the fallback route) and row squared norms.
//
// assign_valu_kernel restates the reference's tensor-core-free kernel
// (flash_kmeans_cuda/csrc/assign/assign_safe.cu:38-81): for each point,
//     dist_k = max(0, x_sq + c_sq[k] - 2 * <x, c_k>)      (assign_common.cuh:33-36)
// with the dot product accumulated in fp32 as one fused multiply-add chain in
// feature order, and the strict-< running minimum that keeps the lowest k on
// ties (assign_common.cuh:23-28).  It serves fp32 inputs, fp16/bf16 with
// D % 8 != 0 or D > 512, and FKC_ASSIGN_FORCE_SAFE (api.cpp:12-25).
//
// Layout: SPLIT adjacent lanes per point (256 / SPLIT points per
// workgroup); lane s of a point scores centroids k = s (mod SPLIT) of each
// tile.  Centroids pass through LDS in 32 x 32 (centroid x feature) fp32
// tiles.  Each lane keeps 32 / SPLIT partial dot products in registers while
// the feature tiles stream past; every (point, centroid) dot product is one
// lane's FMA chain in feature order whatever SPLIT is, so labels do not
// depend on it.  The SPLIT lanes of a point merge with the lowest-index rule
// at the end.  SPLIT > 1 gives small N enough workgroups to fill the chip.
#include "device_util.hpp"
#include "fkc_internal.hpp"

#include <float.h>

namespace fkc {

int launch_assign_mfma(const void* x, const void* c, const float* c_sq,
                       int32_t* ids, int64_t B, int64_t N, int64_t K,
                       int64_t D, int dtype, const int32_t* ctrl,
                       hipStream_t s, hipEvent_t ev0, hipEvent_t ev1,
                       void* ws, size_t ws_bytes);

namespace {

constexpr int VT = 256;   // threads (points) per workgroup
constexpr int VKC = 32;   // centroids per LDS tile
constexpr int VDC = 32;   // features per LDS tile

template <int DT, int SPLIT, bool PREF>
__global__ void __launch_bounds__(VT)
assign_valu_kernel(const typename Elem<DT>::T* __restrict__ x,
                   const typename Elem<DT>::T* __restrict__ c,
                   const float* __restrict__ x_sq,
                   const float* __restrict__ c_sq, int32_t* __restrict__ ids,
                   int N, int K, int D, const int32_t* __restrict__ ctrl) {
  using E = Elem<DT>;
  constexpr int PPW = VT / SPLIT;    // points per workgroup
  constexpr int KPL = VKC / SPLIT;   // centroids per lane per tile
  if (loop_done(ctrl)) return;
  // Rows padded to 36 floats: 16-byte aligned, so the lanes' reads of a
  // row's features become 16-byte loads (one per four FMAs instead of one per
  // FMA; 33-float rows forced 4-byte loads), with at most two-way bank
  // conflicts when lanes read different rows (measured: (262144, 256, 128)
  // fp32 1.00 -> 0.32 ms, (131072, 1024, 128) fp32 2.25 -> 1.92 ms,
  // (100000, 300, 37) fp16 0.100 -> 0.082 ms).
  __shared__ __attribute__((aligned(16))) float tile[VKC][VDC + 4];
  __shared__ float tile_q[VKC];

  const int tid = threadIdx.x;
  const int sl = tid % SPLIT;        // this lane's centroid residue
  const int b = blockIdx.y;
  const int n = blockIdx.x * PPW + tid / SPLIT;
  const bool valid = n < N;
  const typename E::T* xr = x + ((size_t)b * N + (valid ? n : 0)) * D;
  const typename E::T* cb = c + (size_t)b * K * D;

  float xs = 0.f;
  if (x_sq != nullptr) {
    xs = valid ? x_sq[(size_t)b * N + n] : 0.f;
  } else {
    for (int d = 0; d < D; ++d) {
      const float v = E::load(xr[d]);
      xs = fmaf(v, v, xs);
    }
  }

  float best = FLT_MAX;
  int bidx = 0;
  if constexpr (!PREF) {
    // One lane per point (large N: enough waves to hide the loads; the
    // prefetching loop below measured 15% slower at N = 262144) or a
    // partial last feature chunk (computed only over its real features;
    // the prefetching loop would pad it to 32): the plain tile loop.
    for (int k0 = 0; k0 < K; k0 += VKC) {
      float acc[KPL];
  #pragma unroll
      for (int j = 0; j < KPL; ++j) acc[j] = 0.f;
      for (int d0 = 0; d0 < D; d0 += VDC) {
        __syncthreads();
        for (int i = tid; i < VKC * VDC; i += VT) {
          const int kk = i / VDC, dd = i % VDC;
          const int k = k0 + kk, d = d0 + dd;
          tile[kk][dd] = (k < K && d < D) ? E::load(cb[(size_t)k * D + d]) : 0.f;
        }
        if (d0 == 0 && tid < VKC) {
          const int k = k0 + tid;
          tile_q[tid] = k < K ? c_sq[(size_t)b * K + k] : 0.f;
        }
        __syncthreads();
        const int dn = min(VDC, D - d0);
        if (dn == VDC) {
          float xv[VDC];
  #pragma unroll
          for (int dd = 0; dd < VDC; ++dd) xv[dd] = E::load(xr[d0 + dd]);
  #pragma unroll
          for (int j = 0; j < KPL; ++j) {
            const int kk = j * SPLIT + sl;
  #pragma unroll
            for (int dd = 0; dd < VDC; ++dd)
              acc[j] = fmaf(xv[dd], tile[kk][dd], acc[j]);
          }
        } else {
          for (int dd = 0; dd < dn; ++dd) {
            const float xv = E::load(xr[d0 + dd]);
  #pragma unroll
            for (int j = 0; j < KPL; ++j)
              acc[j] = fmaf(xv, tile[j * SPLIT + sl][dd], acc[j]);
          }
        }
      }
  #pragma unroll
      for (int j = 0; j < KPL; ++j) {
        const int kk = j * SPLIT + sl;
        if (k0 + kk < K) {
          float dist = xs + tile_q[kk] - 2.0f * acc[j];
          dist = dist > 0.f ? dist : 0.f;
          if (dist < best) {  // kk rises with j: the first minimum is kept
            best = dist;
            bidx = k0 + kk;
          }
        }
      }
    }
  } else {
  // The (centroid tile, feature chunk) steps run in sequence; the next
  // step's centroid tile (TPT values per thread) and feature chunk are
  // loaded into registers before the current step is computed, so every
  // step's global loads overlap the previous step's arithmetic instead of
  // costing a round trip each.
  constexpr int TPT = VKC * VDC / VT;  // tile values per thread
  static_assert(VKC * VDC % VT == 0, "tile split");
  const int nkt = (K + VKC - 1) / VKC, ndc = (D + VDC - 1) / VDC;
  const int nsteps = nkt * ndc;
  float pt[TPT], pq = 0.f, px[VDC];
  auto fetch = [&](int st) {
    const int k0 = (st / ndc) * VKC, d0 = (st % ndc) * VDC;
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
      const int i = tid + j * VT;
      const int k = k0 + i / VDC, d = d0 + i % VDC;
      pt[j] = (k < K && d < D) ? E::load(cb[(size_t)k * D + d]) : 0.f;
    }
    if (d0 == 0 && tid < VKC)
      pq = k0 + tid < K ? c_sq[(size_t)b * K + k0 + tid] : 0.f;
#pragma unroll
    for (int dd = 0; dd < VDC; ++dd)
      px[dd] = d0 + dd < D ? E::load(xr[d0 + dd]) : 0.f;
  };
  fetch(0);
  float acc[KPL];
  for (int st = 0; st < nsteps; ++st) {
    const int k0 = (st / ndc) * VKC, dc = st % ndc;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
      const int i = tid + j * VT;
      tile[i / VDC][i % VDC] = pt[j];
    }
    if (dc == 0 && tid < VKC) tile_q[tid] = pq;
    float xv[VDC];
#pragma unroll
    for (int dd = 0; dd < VDC; ++dd) xv[dd] = px[dd];
    __syncthreads();
    if (st + 1 < nsteps) fetch(st + 1);
    if (dc == 0) {
#pragma unroll
      for (int j = 0; j < KPL; ++j) acc[j] = 0.f;
    }
    // Features past D are zero in both operands and add nothing.
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      const int kk = j * SPLIT + sl;
#pragma unroll
      for (int dd = 0; dd < VDC; ++dd) acc[j] = fmaf(xv[dd], tile[kk][dd], acc[j]);
    }
    if (dc == ndc - 1) {
#pragma unroll
      for (int j = 0; j < KPL; ++j) {
        const int kk = j * SPLIT + sl;
        if (k0 + kk < K) {
          float dist = xs + tile_q[kk] - 2.0f * acc[j];
          dist = dist > 0.f ? dist : 0.f;
          if (dist < best) {  // kk rises with j: the first minimum is kept
            best = dist;
            bidx = k0 + kk;
          }
        }
      }
    }
  }
  }
  // Merge the SPLIT lanes of this point (adjacent lanes): smaller distance,
  // then smaller index.
#pragma unroll
  for (int off = 1; off < SPLIT; off <<= 1) {
    const float ob = __shfl_xor(best, off, 64);
    const int oi = __shfl_xor(bidx, off, 64);
    if (ob < best || (ob == best && oi < bidx)) {
      best = ob;
      bidx = oi;
    }
  }
  if (valid && sl == 0) ids[(size_t)b * N + n] = bidx;
}

template <int DT>
__global__ void __launch_bounds__(256)
row_sqnorm_kernel(const typename Elem<DT>::T* __restrict__ src,
                  float* __restrict__ out, int64_t rows, int D,
                  const int32_t* __restrict__ ctrl) {
  using E = Elem<DT>;
  if (loop_done(ctrl)) return;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const typename E::T* r = src + row * D;
  // Column order and reduction shared with the finalize kernels.
  const int vec = row_vec(D);
  float acc = 0.f;
  for (int c = vec * lane; c < D; c += vec * 64) {
    for (int v = 0; v < vec; ++v) {
      const float f = E::load(r[c + v]);
      acc = fmaf(f, f, acc);
    }
  }
  acc = row_sum(acc);
  if (lane == 0) out[row] = acc;
}

// Table-resident variant, for tables small enough to sit in LDS whole: the
// K centroid rows and the workgroup's points (rows of D + 4 floats, so every
// row is 16-byte aligned and the 16 lanes of a point read 16 distinct bank
// groups) and the K c_sq values are loaded in one batched round trip, then
// every lane runs its centroids' FMA chains with no further barrier.  The
// chains (one lane per (point, centroid), feature order, starting from 0),
// the distance expression, its clamp, the strict-< scan in rising k and the
// lane merge are those of assign_valu_kernel, so the labels are the same.
// Measured at c1 (1, 4096, 64, 128) fp32, same box: assign 0.0133 -> 0.0108
// -0.0113 ms, Lloyd iteration 0.0332 -> 0.0282-0.0300 ms; a fill in one
// batch of 16 loads per thread and a 4x unrolled feature loop changed
// nothing (the kernel is a few dependent round trips at this size).
constexpr int kValuResidentLds = 64 * 1024;

__host__ __device__ inline int64_t valu_res_bytes(int64_t K, int64_t D,
                                                  int ppw) {
  return (K * (D + 4) + ppw * (D + 4) + K) * 4;
}

// Four consecutive elements (4-element aligned) as fp32.
template <int DT>
__device__ inline float4 load4(const typename Elem<DT>::T* p) {
  using E = Elem<DT>;
  if constexpr (DT == FKC_F32) {
    return *reinterpret_cast<const float4*>(p);
  } else {
    const uint2 r = *reinterpret_cast<const uint2*>(p);
    typename E::T e[4];
    __builtin_memcpy(&e[0], &r, 8);
    return float4{E::load(e[0]), E::load(e[1]), E::load(e[2]), E::load(e[3])};
  }
}

template <int DT, int SPLIT>
__global__ void __launch_bounds__(VT)
assign_valu_resident_kernel(const typename Elem<DT>::T* __restrict__ x,
                            const typename Elem<DT>::T* __restrict__ c,
                            const float* __restrict__ x_sq,
                            const float* __restrict__ c_sq,
                            int32_t* __restrict__ ids, int N, int K, int D,
                            const int32_t* __restrict__ ctrl) {
  using T = typename Elem<DT>::T;
  constexpr int PPW = VT / SPLIT;  // points per workgroup
  constexpr int CH = 8;            // 16-byte loads in flight per thread
  if (loop_done(ctrl)) return;
  extern __shared__ __attribute__((aligned(16))) float s_vr[];
  const int DP = D + 4;
  float* tab = s_vr;              // K rows of DP
  float* pts = tab + K * DP;      // PPW rows of DP
  float* tq = pts + PPW * DP;     // K
  const int tid = threadIdx.x;
  const int sl = tid % SPLIT, pl = tid / SPLIT;
  const int b = blockIdx.y;
  const int n0 = blockIdx.x * PPW;
  const int n = n0 + pl;
  const T* cb = c + (size_t)b * K * D;
  const T* xb = x + (size_t)b * N * D;

  // Fill: every load of a batch is issued before any store.  Groups of four
  // elements never cross a row (D % 4 == 0); points past N load row N-1.
  const int qd = D / 4;
  const int nt = K * qd, np = PPW * qd;
  for (int i0 = 0; i0 < nt + np; i0 += VT * CH) {
    float4 v[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int i = min(i0 + j * VT + tid, nt + np - 1);
      if (i < nt) {
        v[j] = load4<DT>(cb + (size_t)i * 4);
      } else {
        const int r = (i - nt) / qd, q = (i - nt) - r * qd;
        v[j] = load4<DT>(xb + (size_t)min(n0 + r, N - 1) * D + q * 4);
      }
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int i = i0 + j * VT + tid;
      if (i < nt) {
        const int k = i / qd, q = i - k * qd;
        *reinterpret_cast<float4*>(tab + k * DP + q * 4) = v[j];
      } else if (i < nt + np) {
        const int r = (i - nt) / qd, q = (i - nt) - r * qd;
        *reinterpret_cast<float4*>(pts + r * DP + q * 4) = v[j];
      }
    }
  }
  for (int k = tid; k < K; k += VT) tq[k] = c_sq[(size_t)b * K + k];
  __syncthreads();

  const float* xp = pts + pl * DP;
  float xs = 0.f;
  if (x_sq != nullptr) {
    xs = n < N ? x_sq[(size_t)b * N + n] : 0.f;
  } else {
    for (int d = 0; d < D; ++d) {
      const float v = xp[d];
      xs = fmaf(v, v, xs);
    }
  }
  float best = FLT_MAX;
  int bidx = 0;
  constexpr int JB = 4;  // centroids scored together (x read once per 4)
  const int kpl = (K - sl + SPLIT - 1) / SPLIT;  // k = sl + j * SPLIT
  for (int j0 = 0; j0 < kpl; j0 += JB) {
    float acc[JB];
    const float* crow[JB];
#pragma unroll
    for (int jj = 0; jj < JB; ++jj) {
      acc[jj] = 0.f;
      crow[jj] = tab + min(sl + (j0 + jj) * SPLIT, K - 1) * DP;
    }
    for (int d = 0; d < D; d += 4) {
      const float4 xv = *reinterpret_cast<const float4*>(xp + d);
#pragma unroll
      for (int jj = 0; jj < JB; ++jj) {
        const float4 cv = *reinterpret_cast<const float4*>(crow[jj] + d);
        acc[jj] = fmaf(xv.x, cv.x, acc[jj]);
        acc[jj] = fmaf(xv.y, cv.y, acc[jj]);
        acc[jj] = fmaf(xv.z, cv.z, acc[jj]);
        acc[jj] = fmaf(xv.w, cv.w, acc[jj]);
      }
    }
#pragma unroll
    for (int jj = 0; jj < JB; ++jj) {
      if (j0 + jj < kpl) {
        const int k = sl + (j0 + jj) * SPLIT;
        float dist = xs + tq[k] - 2.0f * acc[jj];
        dist = dist > 0.f ? dist : 0.f;
        if (dist < best) {  // k rises with j: the first minimum is kept
          best = dist;
          bidx = k;
        }
      }
    }
  }
#pragma unroll
  for (int off = 1; off < SPLIT; off <<= 1) {
    const float ob = __shfl_xor(best, off, 64);
    const int oi = __shfl_xor(bidx, off, 64);
    if (ob < best || (ob == best && oi < bidx)) {
      best = ob;
      bidx = oi;
    }
  }
  if (n < N && sl == 0) ids[(size_t)b * N + n] = bidx;
}

// PREF (several lanes per point and D a multiple of the 32-feature chunk):
// the prefetching step loop, measured at (1, 4096, 64, 128) fp32 0.0180 ->
// 0.0129 ms and (1, 65536, 1024, 64) fp32 0.338 -> 0.308 ms.
template <int DT, int SPLIT>
int launch_valu_split(const void* x, const void* c, const float* x_sq,
                      const float* c_sq, int32_t* ids, int64_t B, int64_t N,
                      int64_t K, int64_t D, const int32_t* ctrl,
                      hipStream_t s) {
  using T = typename Elem<DT>::T;
  constexpr int PPW = VT / SPLIT;
  dim3 grid((unsigned)((N + PPW - 1) / PPW), (unsigned)B);
  const int64_t rbytes = valu_res_bytes(K, D, PPW);
  if (D % 4 == 0 && rbytes <= kValuResidentLds && resident_override() != 0) {
    hipLaunchKernelGGL((assign_valu_resident_kernel<DT, SPLIT>), grid,
                       dim3(VT), (size_t)rbytes, s, static_cast<const T*>(x),
                       static_cast<const T*>(c), x_sq, c_sq, ids, (int)N,
                       (int)K, (int)D, ctrl);
    return check_launch("assign_valu_resident");
  }
  if (SPLIT > 1 && D % VDC == 0)
    hipLaunchKernelGGL((assign_valu_kernel<DT, SPLIT, SPLIT != 1>), grid,
                       dim3(VT), 0, s, static_cast<const T*>(x),
                       static_cast<const T*>(c), x_sq, c_sq, ids, (int)N,
                       (int)K, (int)D, ctrl);
  else
    hipLaunchKernelGGL((assign_valu_kernel<DT, SPLIT, false>), grid, dim3(VT),
                       0, s, static_cast<const T*>(x),
                       static_cast<const T*>(c), x_sq, c_sq, ids, (int)N,
                       (int)K, (int)D, ctrl);
  return check_launch("assign_valu");
}

// Lanes per point: one while the grid has >= 512 workgroups (2 per CU),
// else the smallest of 4, 8, 16 that gives >= 1024 workgroups.  Two lanes
// per point were never the fastest (measured, ms at 1 / 2 / 4 / 8 / 16 lanes:
// (131072, 1024, 128) fp32 0.94 / 1.93 / 1.05 / 1.05 / 1.63;
// (65536, 1024, 64) fp32 0.43 / 0.53 / 0.27 / 0.29 / 0.43;
// (32768, 512, 128) fp32 0.40 / 0.31 / 0.16 / 0.15 / 0.23;
// (100000, 300, 37) fp16 0.18 / 0.11 / 0.088 / 0.10 / 0.15).
template <int DT>
int launch_valu_t(const void* x, const void* c, const float* x_sq,
                  const float* c_sq, int32_t* ids, int64_t B, int64_t N,
                  int64_t K, int64_t D, const int32_t* ctrl, hipStream_t s) {
  int split = 1;
  if (B * ((N + VT - 1) / VT) < 512) {
    split = 4;
    while (split < 16 && B * ((N * split + VT - 1) / VT) < 1024) split <<= 1;
  }
  switch (split) {
    case 1: return launch_valu_split<DT, 1>(x, c, x_sq, c_sq, ids, B, N, K, D, ctrl, s);
    case 4: return launch_valu_split<DT, 4>(x, c, x_sq, c_sq, ids, B, N, K, D, ctrl, s);
    case 8: return launch_valu_split<DT, 8>(x, c, x_sq, c_sq, ids, B, N, K, D, ctrl, s);
    default: return launch_valu_split<DT, 16>(x, c, x_sq, c_sq, ids, B, N, K, D, ctrl, s);
  }
}

template <int DT>
int launch_rowsq_t(const void* src, float* out, int64_t rows, int64_t D,
                   const int32_t* ctrl, hipStream_t s) {
  using T = typename Elem<DT>::T;
  dim3 grid((unsigned)((rows + 3) / 4));
  hipLaunchKernelGGL((row_sqnorm_kernel<DT>), grid, dim3(256), 0, s,
                     static_cast<const T*>(src), out, rows, (int)D, ctrl);
  return check_launch("row_sqnorm");
}

}  // namespace

int launch_assign(const void* x, const void* c, const float* x_sq,
                  const float* c_sq, int32_t* ids, int64_t B, int64_t N,
                  int64_t K, int64_t D, int dtype, const int32_t* ctrl,
                  hipStream_t s, hipEvent_t ev0, hipEvent_t ev1, void* ws,
                  size_t ws_bytes) {
  if (B == 0 || N == 0) return FKC_OK;
  if (assign_uses_mfma(dtype, D))
    return launch_assign_mfma(x, c, c_sq, ids, B, N, K, D, dtype, ctrl, s,
                              ev0, ev1, ws, ws_bytes);
  // The VALU route marks its span with event records on the stream.
  if (ev0 != nullptr) (void)hipEventRecord(ev0, s);
  int rc = FKC_OK;
  switch (dtype) {
    case FKC_F32:
      rc = launch_valu_t<FKC_F32>(x, c, x_sq, c_sq, ids, B, N, K, D, ctrl, s);
      break;
    case FKC_F16:
      rc = launch_valu_t<FKC_F16>(x, c, x_sq, c_sq, ids, B, N, K, D, ctrl, s);
      break;
    case FKC_BF16:
      rc = launch_valu_t<FKC_BF16>(x, c, x_sq, c_sq, ids, B, N, K, D, ctrl, s);
      break;
    default:
      return fail(FKC_ERR_INVALID, "assign: unknown dtype %d", dtype);
  }
  if (ev1 != nullptr) (void)hipEventRecord(ev1, s);
  return rc;
}

int launch_row_sqnorm(const void* src, float* out, int64_t rows, int64_t D,
                      int dtype, const int32_t* ctrl, hipStream_t s) {
  if (rows == 0) return FKC_OK;
  switch (dtype) {
    case FKC_F32: return launch_rowsq_t<FKC_F32>(src, out, rows, D, ctrl, s);
    case FKC_F16: return launch_rowsq_t<FKC_F16>(src, out, rows, D, ctrl, s);
    case FKC_BF16: return launch_rowsq_t<FKC_BF16>(src, out, rows, D, ctrl, s);
  }
  return fail(FKC_ERR_INVALID, "row_sqnorm: unknown dtype %d", dtype);
}

}  // namespace fkc
