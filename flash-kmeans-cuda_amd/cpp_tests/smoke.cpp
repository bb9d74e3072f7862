// C++ smoke test of the libtorch fkc:: API on PyTorch-ROCm (the counterpart of
// the reference's tests/cpp/smoke.cpp:21-95): assignment against an
// at::matmul reference over many feature widths (odd widths take the fp32
// route), indexed update == materialized update, the finalize formula, the
// stable label sort against at::sort(stable=true), and one Lloyd run.
#include <ATen/ATen.h>

#include <cstdint>
#include <iostream>
#include <stdexcept>
#include <vector>

#include "flash_kmeans_cuda.h"

namespace {

void check(bool ok, const char* msg) {
  if (!ok) throw std::runtime_error(msg);
}

// A device-to-host copy on the current stream waits for all earlier work.
void sync() { (void)at::zeros({1}, at::TensorOptions().device(at::kCUDA)).item<float>(); }

at::Tensor reference_assign(const at::Tensor& x, const at::Tensor& c) {
  at::Tensor xf = x.to(at::kDouble), cf = c.to(at::kDouble);
  at::Tensor dist = xf.pow(2).sum(-1).unsqueeze(-1) + cf.pow(2).sum(-1).unsqueeze(1) -
                    2.0 * at::matmul(xf, cf.transpose(1, 2));
  return std::get<1>(dist.min(-1)).to(at::kInt);
}

void test_assign(int64_t D) {
  const int64_t B = 1, N = 512, K = 64;
  auto opts = at::TensorOptions().device(at::kCUDA).dtype(at::kHalf);
  at::Tensor x = at::randn({B, N, D}, opts).contiguous();
  at::Tensor c = at::randn({B, K, D}, opts).contiguous();
  at::Tensor x_sq = x.to(at::kFloat).pow(2).sum(-1).contiguous();
  at::Tensor c_sq = c.to(at::kFloat).pow(2).sum(-1).contiguous();
  at::Tensor ids = fkc::euclid_assign(x, c, x_sq, c_sq);
  sync();
  at::Tensor ref = reference_assign(x, c);
  check(ids.sizes() == at::IntArrayRef({B, N}), "assign output shape mismatch");
  check(ids.scalar_type() == at::kInt, "assign output dtype mismatch");
  const double dis = ids.ne(ref).to(at::kFloat).mean().item<double>();
  std::cout << "assign D=" << D << " disagreement=" << dis << "\n";
  check(dis < 0.01, "assign disagreement exceeds 1%");
}

void test_update_finalize(int64_t D) {
  const int64_t B = 1, N = 512, K = 16;
  auto xo = at::TensorOptions().device(at::kCUDA).dtype(at::kFloat);
  auto io = at::TensorOptions().device(at::kCUDA).dtype(at::kInt);
  at::Tensor x = at::randn({B, N, D}, xo).contiguous();
  at::Tensor ids = at::randint(K, {B, N}, io).contiguous();
  auto sp = at::sort(ids, /*stable=*/true, 1, false);
  at::Tensor sorted_ids = std::get<0>(sp).contiguous();
  at::Tensor sorted_idx = std::get<1>(sp).to(at::kInt).contiguous();
  at::Tensor x_sorted =
      x.gather(1, sorted_idx.to(at::kLong).unsqueeze(-1).expand({B, N, D})).contiguous();

  at::Tensor sums = at::empty({B, K, D}, xo), counts = at::empty({B, K}, io);
  fkc::centroid_update_sorted(x_sorted, sorted_ids, sums, counts);
  at::Tensor sums_i = at::empty_like(sums), counts_i = at::empty_like(counts);
  fkc::centroid_update_sorted_indexed(x, sorted_idx, sorted_ids, sums_i, counts_i);
  sync();
  check(sums.equal(sums_i), "indexed update sums differ from materialized");
  check(counts.equal(counts_i), "indexed update counts differ from materialized");
  check(counts.sum().item<int64_t>() == N, "counts do not sum to N");
  at::Tensor ref_sums = at::zeros({B, K, D}, xo).index_add_(1, ids[0].to(at::kLong), x);
  check(at::allclose(sums, ref_sums, 1e-4, 1e-4), "sums differ from index_add_");

  auto [fk_sorted, fk_perm] = fkc::label_sort(ids, K);
  sync();
  check(fk_sorted.equal(sorted_ids) && fk_perm.equal(sorted_idx), "label_sort != stable sort");

  at::Tensor old = at::randn({B, K, D}, xo).contiguous();
  at::Tensor fin = fkc::centroid_finalize(sums, counts, old);
  sync();
  at::Tensor ref = at::where(counts.unsqueeze(-1).gt(0),
                             sums / counts.clamp_min(1).to(at::kFloat).unsqueeze(-1), old);
  check(at::allclose(fin, ref, 1e-6, 1e-6), "finalize output mismatch");
  std::cout << "update/finalize D=" << D << " passed\n";
}

void test_lloyd() {
  auto opts = at::TensorOptions().device(at::kCUDA).dtype(at::kHalf);
  at::Tensor x = at::randn({2, 4096, 128}, opts);
  at::Tensor init = x.narrow(1, 0, 64).contiguous();
  at::Tensor init_copy = init.clone();
  auto [ids, cents, n] = fkc::batch_kmeans_euclid(x, 64, 5, 0.0, init);
  sync();
  check(n == 5, "n_iters != max_iters with tol=0");
  check(ids.sizes() == at::IntArrayRef({2, 4096}) && cents.sizes() == init.sizes(), "shapes");
  check(ids.min().item<int>() >= 0 && ids.max().item<int>() < 64, "ids out of range");
  check(init.equal(init_copy), "init_centroids modified");
  std::cout << "batch_kmeans_euclid passed\n";
}

}  // namespace

int main() {
  try {
    check(at::hasCUDA(), "no GPU visible to libtorch");
    at::manual_seed(0);
    for (int64_t D : std::vector<int64_t>{1, 7, 16, 31, 32, 48, 64, 96, 128, 256, 257})
      test_assign(D);
    for (int64_t D : std::vector<int64_t>{1, 7, 16, 31, 32, 64, 128, 257}) test_update_finalize(D);
    test_lloyd();
    bool threw = false;
    try {
      fkc::euclid_assign(at::randn({1, 4, 8}), at::randn({1, 2, 8}), at::randn({1, 4}),
                         at::randn({1, 2}));
    } catch (const c10::Error&) {
      threw = true;
    }
    check(threw, "CPU tensors were not rejected");
    std::cout << "flash_kmeans_cuda C++ smoke test passed\n";
    return 0;
  } catch (const std::exception& e) {
    std::cerr << "flash_kmeans_cuda C++ smoke test failed: " << e.what() << "\n";
    return 1;
  }
}
