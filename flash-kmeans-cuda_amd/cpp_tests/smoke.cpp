// fkc_cpp_smoke: end-to-end check of the libtorch fkc:: API on PyTorch-ROCm.
//
// It covers what the reference's C++ smoke test covers (tests/cpp/smoke.cpp:
// assignment over the same feature widths, the sorted update read directly
// and through the permutation, the finalize rule), checked more strictly:
//   assign   every label is the nearest centroid by exact fp64 distance
//            (at::cdist), except where two centroids are closer than fp32
//            can tell apart: gap <= 2^-16 * (|x|^2 + |c|^2);
//   update   permutation-read and row-read sums are the same bits, counts
//            equal at::bincount, sums match index_add_ in fp32;
//   sort     fkc::label_sort equals at::sort(stable=true);
//   finalize mean where the count is positive, the old row elsewhere;
// plus a short Lloyd run and the rejection of CPU tensors.  Every check is
// counted; the process exits non-zero if any fails.
#include <ATen/ATen.h>

#include <cmath>
#include <cstdio>
#include <string>

#include "flash_kmeans_cuda.h"

namespace {

struct Tally {
  int checks = 0;
  int failures = 0;
  void expect(bool ok, const std::string& what) {
    ++checks;
    if (!ok) {
      ++failures;
      std::printf("  FAILED: %s\n", what.c_str());
    }
  }
};

at::TensorOptions gpu(at::ScalarType t) {
  return at::TensorOptions().device(at::kCUDA).dtype(t);
}

// Waits for every queued kernel on the current stream (the scalar read back
// is ordered after them).
void drain() { (void)at::ones({1}, gpu(at::kFloat)).sum().item<float>(); }

at::Tensor sq_norms(const at::Tensor& t) {
  return t.to(at::kFloat).pow(2).sum(-1).contiguous();
}

// Labels from fkc::euclid_assign against exact nearest centroids.
void section_assign(Tally& t) {
  const int64_t widths[] = {1, 7, 16, 31, 32, 48, 64, 96, 128, 256, 257};
  for (int64_t D : widths) {
    const std::string tag = "assign D=" + std::to_string(D);
    at::Tensor pts = at::randn({1, 512, D}, gpu(at::kHalf));
    at::Tensor cen = at::randn({1, 64, D}, gpu(at::kHalf));
    at::Tensor got = fkc::euclid_assign(pts, cen, sq_norms(pts), sq_norms(cen));
    drain();
    t.expect(got.scalar_type() == at::kInt && got.dim() == 2 && got.size(0) == 1 &&
                 got.size(1) == 512,
             tag + ": int32 labels of shape (1, 512)");
    at::Tensor pd = pts.to(at::kDouble), cd = cen.to(at::kDouble);
    at::Tensor d2 = at::cdist(pd, cd).pow(2);                     // (1, 512, 64)
    at::Tensor nearest = std::get<0>(d2.min(-1));
    at::Tensor mine = d2.gather(-1, got.to(at::kLong).unsqueeze(-1)).squeeze(-1);
    at::Tensor cn = cd.pow(2).sum(-1);                            // (1, 64)
    at::Tensor slack = (pd.pow(2).sum(-1) + cn.gather(1, got.to(at::kLong))) *
                       std::ldexp(1.0, -16);
    const int64_t far = (mine - nearest).gt(slack).sum().item<int64_t>();
    const int64_t flips = got.to(at::kLong).ne(std::get<1>(d2.min(-1))).sum().item<int64_t>();
    std::printf("%s: %lld labels off the exact nearest (all near-ties: %s)\n", tag.c_str(),
                (long long)flips, far == 0 ? "yes" : "no");
    t.expect(far == 0, tag + ": labels are nearest up to fp32 near-ties");
  }
}

// Sorted update (both reads), label sort and finalize.
void section_update(Tally& t) {
  const int64_t widths[] = {1, 7, 16, 31, 32, 64, 128, 257};
  const int64_t N = 512, K = 16;
  for (int64_t D : widths) {
    const std::string tag = "update D=" + std::to_string(D);
    at::Tensor pts = at::randn({1, N, D}, gpu(at::kFloat));
    at::Tensor lab = at::randint(K, {1, N}, gpu(at::kInt));
    auto by_label = at::sort(lab, /*stable=*/true, /*dim=*/1, /*descending=*/false);
    at::Tensor keys = std::get<0>(by_label).contiguous();
    at::Tensor perm = std::get<1>(by_label).to(at::kInt).contiguous();
    at::Tensor rows = pts.index_select(1, perm[0].to(at::kLong)).contiguous();

    at::Tensor s_rows = at::full({1, K, D}, 7.0, gpu(at::kFloat));  // zeroed by the API
    at::Tensor n_rows = at::full({1, K}, 7, gpu(at::kInt));
    fkc::centroid_update_sorted(rows, keys, s_rows, n_rows);
    at::Tensor s_perm = at::empty({1, K, D}, gpu(at::kFloat));
    at::Tensor n_perm = at::empty({1, K}, gpu(at::kInt));
    fkc::centroid_update_sorted_indexed(pts, perm, keys, s_perm, n_perm);
    drain();
    t.expect(s_rows.equal(s_perm), tag + ": permutation-read sums == row-read sums (bits)");
    t.expect(n_rows.equal(n_perm), tag + ": permutation-read counts == row-read counts");
    at::Tensor hist = at::bincount(lab[0].to(at::kLong), {}, K).to(at::kInt);
    t.expect(n_perm[0].equal(hist), tag + ": counts == bincount");
    at::Tensor want = at::zeros({K, D}, gpu(at::kFloat)).index_add_(0, lab[0].to(at::kLong),
                                                                    pts[0]);
    t.expect(at::allclose(s_perm[0], want, 1e-5, 1e-4), tag + ": sums == index_add_");

    auto mine = fkc::label_sort(lab, K);
    drain();
    t.expect(std::get<0>(mine).equal(keys) && std::get<1>(mine).equal(perm),
             tag + ": fkc::label_sort == stable at::sort");

    at::Tensor prev = at::randn({1, K, D}, gpu(at::kFloat));
    at::Tensor fin = fkc::centroid_finalize(s_perm, n_perm, prev);
    drain();
    at::Tensor n = n_perm.unsqueeze(-1);
    at::Tensor rule = at::where(n.gt(0), s_perm / n.clamp_min(1).to(at::kFloat), prev);
    t.expect(at::allclose(fin, rule, 1e-6, 1e-6), tag + ": finalize rule");
  }
}

void section_lloyd(Tally& t) {
  at::Tensor pts = at::randn({2, 4096, 128}, gpu(at::kHalf));
  at::Tensor start = pts.narrow(1, 0, 64).contiguous();
  at::Tensor kept = start.clone();
  auto out = fkc::batch_kmeans_euclid(pts, 64, 5, 0.0, start);
  drain();
  const at::Tensor& lab = std::get<0>(out);
  const at::Tensor& cen = std::get<1>(out);
  t.expect(std::get<2>(out) == 5, "lloyd: tol = 0 runs every iteration");
  t.expect(lab.size(0) == 2 && lab.size(1) == 4096 && cen.sizes() == start.sizes(),
           "lloyd: output shapes");
  t.expect(lab.min().item<int>() >= 0 && lab.max().item<int>() < 64, "lloyd: labels in range");
  t.expect(start.equal(kept), "lloyd: initial centroids untouched");
  std::printf("lloyd: 5 iterations at (2, 4096, 64, 128) fp16 done\n");
}

void section_rejects_cpu(Tally& t) {
  bool rejected = false;
  try {
    at::Tensor p = at::randn({1, 4, 8}), c = at::randn({1, 2, 8});
    (void)fkc::euclid_assign(p, c, sq_norms(p), sq_norms(c));
  } catch (const c10::Error&) {
    rejected = true;
  }
  t.expect(rejected, "host tensors raise c10::Error");
}

}  // namespace

int main() {
  Tally t;
  if (!at::hasCUDA()) {
    std::printf("fkc_cpp_smoke: libtorch sees no GPU\n");
    return 2;
  }
  at::manual_seed(0);
  try {
    section_assign(t);
    section_update(t);
    section_lloyd(t);
    section_rejects_cpu(t);
  } catch (const std::exception& e) {
    std::printf("fkc_cpp_smoke: exception: %s\n", e.what());
    return 1;
  }
  std::printf("fkc_cpp_smoke: %d checks, %d failed\n", t.checks, t.failures);
  return t.failures == 0 ? 0 : 1;
}
