// consumer_smoke: a program built only against the *installed* package
// (find_package(flash_kmeans_cuda CONFIG), target
// flash_kmeans_cuda::flash_kmeans_cuda), as a downstream project would use
// it.  It includes <flash_kmeans_cuda/flash_kmeans_cuda.h> from the install
// tree, labels random fp16 points (every label must be the exact fp64
// nearest centroid up to fp32 near-ties), runs five Lloyd iterations, and
// reads /proc/self/maps to make sure torch and the package share one HIP
// runtime.  The reference ships the same kind of consumer with its CMake
// package (tests/cpp/consumer/).
#include <ATen/ATen.h>

#include <flash_kmeans_cuda/flash_kmeans_cuda.h>

#include <cmath>
#include <cstdio>
#include <fstream>
#include <set>
#include <string>

namespace {

// Distinct libamdhip64 files mapped into this process.
int count_hip_runtimes() {
  std::ifstream maps("/proc/self/maps");
  std::set<std::string> seen;
  for (std::string line; std::getline(maps, line);) {
    const size_t at = line.find('/');
    if (at != std::string::npos && line.find("libamdhip64.so", at) != std::string::npos)
      seen.insert(line.substr(at));
  }
  return static_cast<int>(seen.size());
}

int run() {
  const int64_t N = 512, K = 64, D = 64;
  const auto half = at::TensorOptions().device(at::kCUDA).dtype(at::kHalf);
  at::Tensor pts = at::randn({1, N, D}, half);
  at::Tensor cen = at::randn({1, K, D}, half);
  at::Tensor lab = fkc::euclid_assign(pts, cen, pts.to(at::kFloat).pow(2).sum(-1),
                                      cen.to(at::kFloat).pow(2).sum(-1));
  if (lab.scalar_type() != at::kInt || lab.size(0) != 1 || lab.size(1) != N) {
    std::printf("consumer: labels are not int32 (1, %lld)\n", (long long)N);
    return 1;
  }
  at::Tensor d2 = at::cdist(pts.to(at::kDouble), cen.to(at::kDouble)).pow(2);
  at::Tensor gap = d2.gather(-1, lab.to(at::kLong).unsqueeze(-1)).squeeze(-1) -
                   std::get<0>(d2.min(-1));
  at::Tensor slack = (pts.to(at::kDouble).pow(2).sum(-1) +
                      cen.to(at::kDouble).pow(2).sum(-1).gather(1, lab.to(at::kLong))) *
                     std::ldexp(1.0, -16);
  const int64_t wrong = gap.gt(slack).sum().item<int64_t>();
  if (wrong != 0) {
    std::printf("consumer: %lld labels are not the nearest centroid\n", (long long)wrong);
    return 1;
  }

  auto res = fkc::batch_kmeans_euclid(pts, K, 5, 0.0, cen);
  const at::Tensor& lloyd_lab = std::get<0>(res);
  const at::Tensor& lloyd_cen = std::get<1>(res);
  if (std::get<2>(res) != 5 || lloyd_cen.sizes() != cen.sizes() ||
      lloyd_cen.scalar_type() != at::kHalf || lloyd_lab.min().item<int32_t>() < 0 ||
      lloyd_lab.max().item<int32_t>() >= K) {
    std::printf("consumer: Lloyd run returned unexpected results\n");
    return 1;
  }

  const int runtimes = count_hip_runtimes();
  std::printf("consumer: %lld labels checked, Lloyd ran 5 iterations, hip_runtimes=%d\n",
              (long long)N, runtimes);
  if (runtimes != 1) return 1;
  std::printf("consumer: installed package works\n");
  return 0;
}

}  // namespace

int main() {
  if (!at::hasCUDA()) {
    std::printf("consumer: libtorch sees no GPU\n");
    return 2;
  }
  at::manual_seed(0);
  try {
    return run();
  } catch (const std::exception& e) {
    std::printf("consumer: exception: %s\n", e.what());
    return 1;
  }
}
