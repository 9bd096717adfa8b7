// Launchers of the codec kernels (codec.hip): quantizer, 16-bit packing, row lookup.
#pragma once

#include "common.h"

namespace efh {

// w: row-major FP32 [rows][cols] (device); out: rows * row_bytes(qtype, cols) bytes (device).
int launch_quantize(int qtype, const float* w, size_t rows, size_t cols, int search, void* out, hipStream_t s);
// out[b][0..cols) = row ids[b] of W as FP32, for b < batch.
int launch_rows_f32(const ef_hip_weight_s* W, const int32_t* ids, int batch, float* out, size_t ldo, hipStream_t s);

// out[i] = mean + scale * N(0,1) from Philox4x32-10 + Box-Muller, deterministic in (seed, offset, i).
int launch_fill_normal(float* out, size_t n, uint64_t seed, uint64_t offset, float mean, float scale, hipStream_t s);

}  // namespace efh
