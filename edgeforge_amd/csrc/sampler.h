// Launchers of the selection kernels (sampler.hip): argmax, the sampler and its device RNG.
#pragma once

#include "common.h"

namespace efh {

constexpr size_t kRngStateBytes = 2560;  // std::mt19937_64 state (312 words + index), padded

// Workspace bytes one sequence of `vocab` logits needs (work copy, probabilities, sort keys).
size_t sample_workspace_stride(int vocab);
int launch_rng_seed(void* rng, const uint64_t* seeds_dev, int batch, hipStream_t s);
int launch_argmax(const float* x, int n, long ld, int batch, int32_t* out, hipStream_t s);

// Device-resident step state of the decode engine, advanced by the kernel that picks the token.
struct StepArgs {
  int32_t* next;        // [batch] picked ids
  int32_t* hist;        // [batch][hist_ld] token history (prompt + generated)
  long hist_ld;
  int32_t* hist_len;    // [batch]
  int32_t* out;         // [batch][out_ld] generated ids
  long out_ld;
  const int32_t* n_prompt;
  int32_t* pos;         // current position (shared by the batch)
  uint32_t* counter;    // zero between steps
};
// argmax per sequence, then the step bookkeeping (pos advances once for the batch).
int launch_argmax_finish(const float* x, int n, long ld, int batch, const StepArgs& f, hipStream_t s);
// ws: batch * sample_workspace_stride(vocab) bytes of device memory.
// With eos_p: also P(eos_id) under softmax of the raw logits per sequence (prob_of, src/chat.cpp:35-42).
int launch_sample(const float* logits, int vocab, int batch, long ld, const ef_hip_sampler_config& cfg,
                  const int32_t* hist, const int32_t* hist_len, long hist_ld, void* rng, int32_t* out, void* ws,
                  hipStream_t s, int eos_id = -1, double* eos_p = nullptr);
// y[i] = exp(x[i]), the sampler's softmax-term call.
int launch_exp(const double* x, double* y, size_t n, hipStream_t s);
// std::mt19937_64::discard(k) on every sequence's state.
int launch_rng_discard(void* rng, int batch, int k, hipStream_t s);

}  // namespace efh
