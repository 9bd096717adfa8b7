// Launchers of the packed GEMV kernels (gemv.hip), shared by the C-ABI and the decode engine.
#pragma once

#include "common.h"

namespace efh {

enum Epilogue : int { kEpiStore = 0, kEpiResidual = 1, kEpiSwiglu = 2 };

// One product of a launch.  For kEpiSwiglu, W is the gate matrix and W2 the up matrix (same shape
// and type); y = silu(W x) * (W2 x).  For kEpiResidual, y += W x.  Otherwise y = W x.
struct GemvJob {
  const ef_hip_weight_s* W = nullptr;
  const ef_hip_weight_s* W2 = nullptr;
  const float* x = nullptr;
  float* y = nullptr;
  size_t ldx = 0, ldy = 0;  // per-job batch strides in floats; 0 = the launch's ldx / ldy
};

// All jobs of one launch share cols, the epilogue and the optional input RMSNorm (norm_w != null:
// x' = norm_w * (x * rsqrt(mean(x^2) + eps)), kern::rmsnorm order).  batch sequences with row
// strides ldx / ldy.  Enqueues on `stream`; returns an EF_HIP_* status.
int launch_gemv(const GemvJob* jobs, int n_jobs, int epi, const float* norm_w, float eps, int batch, size_t ldx,
                size_t ldy, hipStream_t stream);

}  // namespace efh
