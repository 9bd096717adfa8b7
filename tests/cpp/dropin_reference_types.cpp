// Compiled against the reference's own headers (include/ef/qkernels.h, include/ef/sampler.h): the
// Level-1 drop-in, a Backend::Hip branch of each ef::kern entry point, written with the reference's
// types and forwarding to ef::hip.  It only has to compile and link (no GPU is needed): it proves the
// shim's signatures accept the reference's WeightView, MatvecJob, SamplerConfig and ThreadPool as
// they are, and that nothing is left unresolved beyond the reference's own sources.
#include <cstdint>
#include <cstdio>
#include <type_traits>
#include <vector>

#include "ef/qkernels.h"
#include "ef/sampler.h"
#include "ef_hip_kern.hpp"

// the shim saw the reference's declarations, not its standalone copies
static_assert(std::is_same_v<decltype(ef::kern::MatvecJob::W), const ef::WeightView*>);
static_assert(std::is_same_v<decltype(ef::SamplerConfig::seed), std::uint64_t>);

namespace patched {  // what src/qkernels.cpp:275-297 and src/sampler.cpp:13 would call
void matvec(float* y, const ef::WeightView& W, const float* x, ef::ThreadPool* pool) noexcept {
  ef::hip::matvec(y, W, x, pool);
}
void matvec_jobs(const ef::kern::MatvecJob* jobs, std::size_t n, ef::ThreadPool* pool) noexcept {
  ef::hip::matvec_jobs(jobs, n, pool);
}
void matvec_rows(float* y, const ef::WeightView& W, const float* x, std::size_t b, std::size_t e) noexcept {
  ef::hip::matvec_rows(y, W, x, b, e);
}
void row_f32(float* out, const ef::WeightView& W, std::size_t r) noexcept { ef::hip::row_f32(out, W, r); }
std::int32_t sample(const ef::SamplerConfig& cfg, const std::vector<float>& logits,
                    const std::vector<std::int32_t>& history) {
  ef::hip::Sampler s(cfg);
  return s.sample(logits.data(), logits.size(), history);
}
}  // namespace patched

int main(int argc, char**) {
  // reached only when asked to (argc > 1) and a GPU is present; the test only links this program
  if (argc > 1 && ef::hip::available()) {
    std::vector<std::uint8_t> w(18 * 2, 0);
    const ef::WeightView W{ef::QType::Q4_0, w.data(), 2, 32};
    std::vector<float> x(32, 1.0f), y(2);
    patched::matvec(y.data(), W, x.data(), nullptr);
    ef::hip::throw_if_error();
  }
  std::printf("linked: %zu bytes per Q4_0 row of 32\n", ef::WeightView{ef::QType::Q4_0, nullptr, 1, 32}.row_bytes());
  return 0;
}
