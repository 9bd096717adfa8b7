// Launchers of the selection kernels (sampler.hip): argmax, the sampler and its device RNG.
#pragma once

#include "common.h"

namespace efh {

constexpr size_t kRngStateBytes = 2560;  // std::mt19937_64 state (312 words + index), padded

// Workspace bytes one sequence of `vocab` logits needs (work copy, probabilities, sort keys).
size_t sample_workspace_stride(int vocab);
int launch_rng_seed(void* rng, const uint64_t* seeds_dev, int batch, hipStream_t s);
int launch_argmax(const float* x, int n, long ld, int batch, int32_t* out, hipStream_t s);
// ws: batch * sample_workspace_stride(vocab) bytes of device memory.
int launch_sample(const float* logits, int vocab, int batch, long ld, const ef_hip_sampler_config& cfg,
                  const int32_t* hist, const int32_t* hist_len, long hist_ld, void* rng, int32_t* out, void* ws,
                  hipStream_t s);

}  // namespace efh
