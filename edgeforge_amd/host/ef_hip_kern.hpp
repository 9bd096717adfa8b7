// C++20 face of the MI355X hot path with EdgeForge's own call signatures.
//
// namespace ef::hip mirrors ef::kern's packed-GEMV entry points and ef::Sampler
// (include/ef/qkernels.h:28-78, include/ef/sampler.h:13-35, include/ef/kernels.h:57) so that the
// reference's Transformer::forward (src/model.cpp:184-276) and ChatSession::reply
// (src/chat.cpp:216) can dispatch to the GPU with a Backend::Hip branch and no other change.
// Everything here talks to the GPU only through the C-ABI of include/ef_hip.h.
//
// Pointers: x / y / logits may be host or device addresses.  Device addresses (from ef_hip_malloc)
// are used in place; host addresses are staged through device buffers owned by this layer, which
// is correct but pays a PCIe round trip per call (keep activations on the device for speed).
// Weights: a WeightView's bytes are uploaded once, on first use, and looked up by
// (data, type, rows, cols) afterwards; views must stay valid (they do: they point into the Model's
// mapping).
//
// Errors: the GEMV entry points are noexcept, as in the reference, so a failed call records a
// sticky error (the first one wins) that throw_if_error() rethrows as ef::Error - call it where
// the reference would surface a failure, e.g. at the end of Transformer::forward.  Sampler::sample
// and set_device throw directly, like the reference's configuration errors.
#pragma once

#include <cstddef>
#include <cstdint>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#if !defined(EF_HIP_STANDALONE) && __has_include("ef/qkernels.h") && __has_include("ef/sampler.h")
#include "ef/error.h"
#include "ef/qkernels.h"
#include "ef/sampler.h"
#else
// Standalone build: the reference's public types, declared with the same names, layout and
// meaning (include/ef/quant.h:35, include/ef/qkernels.h:28-34, :70-74, include/ef/sampler.h:13-19,
// include/ef/error.h:11-13) so code written against the reference compiles unchanged.
namespace ef {
enum class QType : std::uint8_t { F32, F16, BF16, Q8_0, Q4_0 };
struct WeightView {
  QType type = QType::BF16;
  const std::uint8_t* data = nullptr;
  std::size_t rows = 0, cols = 0;
  std::size_t row_bytes() const;
  std::uint64_t bytes() const { return static_cast<std::uint64_t>(row_bytes()) * rows; }
};
class ThreadPool;
namespace kern {
struct MatvecJob {
  float* y;
  const WeightView* W;
  const float* x;
};
}  // namespace kern
struct SamplerConfig {
  float temperature = 0.0f;
  int top_k = 0;
  float top_p = 1.0f;
  float repetition_penalty = 1.0f;
  std::uint64_t seed = 0;
};
class Error : public std::runtime_error {
 public:
  using std::runtime_error::runtime_error;
};
}  // namespace ef
#endif

namespace ef::hip {

// Selects and initialises the GPU (throws ef::Error when none is usable).  Called implicitly by
// the first GEMV / sampler call with device 0.
void set_device(int device);
bool available() noexcept;  // a gfx950 device can be initialised

// ---- packed GEMV: same signatures and meaning as ef::kern (include/ef/qkernels.h:47-78) --------
// The ThreadPool argument is accepted for signature compatibility and ignored: the GPU splits rows
// across its own compute units.
void matvec(float* y, const WeightView& W, const float* x, ThreadPool* pool = nullptr) noexcept;
void matvec_jobs(const kern::MatvecJob* jobs, std::size_t n_jobs, ThreadPool* pool) noexcept;
void matvec_rows(float* y, const WeightView& W, const float* x, std::size_t begin, std::size_t end) noexcept;
void matvec_q4_0(float* y, const std::uint8_t* W, const float* x, std::size_t rows, std::size_t cols) noexcept;
void matvec_q8_0(float* y, const std::uint8_t* W, const float* x, std::size_t rows, std::size_t cols) noexcept;
float dot_q4_0(const std::uint8_t* row, const float* x, std::size_t n) noexcept;
float dot_q8_0(const std::uint8_t* row, const float* x, std::size_t n) noexcept;
void row_f32(float* out, const WeightView& W, std::size_t r) noexcept;
std::size_t argmax(const float* x, std::size_t n) noexcept;  // kern::argmax (include/ef/kernels.h:57)

// Sticky error of the noexcept entry points (empty when none).
std::string last_error();
void throw_if_error();  // throws ef::Error with the first recorded failure, then clears it
void clear_error() noexcept;

// Device buffers for callers that keep activations resident (the fast path).
float* device_alloc(std::size_t floats);
void device_free(void* p) noexcept;
void upload(float* dev, const float* host, std::size_t floats);
void download(float* host, const float* dev, std::size_t floats);

// ---- sampler: ef::Sampler (include/ef/sampler.h:21-35, src/sampler.cpp:13-70) -----------------
// Same constructor, same sample() contract: logits are copied (never modified), history feeds the
// repetition penalty, the RNG is std::mt19937_64 seeded with cfg.seed and advanced once per call
// exactly when temperature > 0; the id equals the reference's on identical logits.  The RNG
// state lives on the device; logits may be host or device pointers.
class Sampler {
 public:
  explicit Sampler(const SamplerConfig& cfg);
  ~Sampler();
  Sampler(const Sampler&) = delete;
  Sampler& operator=(const Sampler&) = delete;
  std::int32_t sample(const float* logits, std::size_t vocab, const std::vector<std::int32_t>& history);
  const SamplerConfig& config() const noexcept { return cfg_; }

 private:
  SamplerConfig cfg_;
  void* rng_ = nullptr;     // device std::mt19937_64 state
  void* ws_ = nullptr;      // device workspace
  std::size_t ws_vocab_ = 0;
  float* logits_ = nullptr;  // device staging for host logits
  std::size_t logits_cap_ = 0;
  std::int32_t* hist_ = nullptr;
  std::size_t hist_cap_ = 0;
  std::int32_t* out_ = nullptr;
};

}  // namespace ef::hip
