// Consumer of the installed flash_kmeans_cuda package (counterpart of the
// reference's tests/cpp/consumer/main.cpp): includes the installed header,
// links the exported target, assigns against an at::matmul reference, runs a
// short Lloyd loop, and checks that the process mapped exactly one HIP
// runtime (torch's and the library's must be the same).
#include <ATen/ATen.h>

#include <flash_kmeans_cuda/flash_kmeans_cuda.h>

#include <fstream>
#include <iostream>
#include <set>
#include <stdexcept>
#include <string>

namespace {

void check(bool ok, const char* msg) {
  if (!ok) throw std::runtime_error(msg);
}

int hip_runtimes_mapped() {
  std::ifstream maps("/proc/self/maps");
  std::set<std::string> files;
  std::string line;
  while (std::getline(maps, line)) {
    const auto pos = line.find('/');
    if (pos == std::string::npos) continue;
    const std::string path = line.substr(pos);
    if (path.find("libamdhip64.so") != std::string::npos) files.insert(path);
  }
  return static_cast<int>(files.size());
}

}  // namespace

int main() {
  try {
    check(at::hasCUDA(), "no GPU visible to libtorch");
    at::manual_seed(0);
    constexpr int64_t B = 1, N = 512, K = 64, D = 64;
    auto opts = at::TensorOptions().device(at::kCUDA).dtype(at::kHalf);
    at::Tensor x = at::randn({B, N, D}, opts).contiguous();
    at::Tensor c = at::randn({B, K, D}, opts).contiguous();
    at::Tensor x_sq = x.to(at::kFloat).pow(2).sum(-1).contiguous();
    at::Tensor c_sq = c.to(at::kFloat).pow(2).sum(-1).contiguous();

    at::Tensor ids = fkc::euclid_assign(x, c, x_sq, c_sq);
    check(ids.sizes() == at::IntArrayRef({B, N}), "assign output shape mismatch");
    check(ids.scalar_type() == at::kInt, "assign output dtype mismatch");

    at::Tensor xf = x.to(at::kDouble), cf = c.to(at::kDouble);
    at::Tensor dist = xf.pow(2).sum(-1).unsqueeze(-1) + cf.pow(2).sum(-1).unsqueeze(1) -
                      2.0 * at::matmul(xf, cf.transpose(1, 2));
    at::Tensor ref = std::get<1>(dist.min(-1)).to(at::kInt);
    const int64_t agree = ids.eq(ref).sum().item<int64_t>();
    check(agree >= N - 2, "assign disagrees with the matmul reference");

    auto [lab, cents, n_iters] = fkc::batch_kmeans_euclid(x, K, 5, 0.0, c);
    check(n_iters == 5, "Lloyd loop did not run 5 iterations");
    check(cents.sizes() == c.sizes() && cents.scalar_type() == at::kHalf,
          "Lloyd centroids shape/dtype mismatch");
    check(lab.min().item<int32_t>() >= 0 && lab.max().item<int32_t>() < K,
          "Lloyd labels out of range");

    const int runtimes = hip_runtimes_mapped();
    check(runtimes == 1, "more than one HIP runtime mapped in the process");
    std::cout << "consumer smoke ids[0,0]=" << ids[0][0].item<int32_t>()
              << " agree=" << agree << "/" << N << " hip_runtimes=" << runtimes << "\n";
    std::cout << "flash_kmeans_cuda installed C++ consumer smoke passed\n";
    return 0;
  } catch (const std::exception& e) {
    std::cerr << "flash_kmeans_cuda installed C++ consumer smoke failed: " << e.what() << "\n";
    return 1;
  }
}
