// Launchers of the packed GEMV kernels (gemv.hip), shared by the C-ABI and the decode engine.
#pragma once

#include "afrag.h"
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

// Matrix-core path for batches of 2 or more sequences (gemv_mfma.hip).  Sets *taken when it enqueued
// the launches; otherwise the caller uses the vector-ALU kernels.  ws (>= gemv_mfma_workspace_bytes
// for the same launch) holds the prepared activation fragments and the split-K partial sums;
// without it the launch allocates stream-ordered memory.  0 when the launch does not take this path.
size_t gemv_mfma_workspace_bytes(const GemvJob* jobs, int n_jobs, int epi, int batch, size_t ldx);
// Rows (sequences) one matrix-core launch covers; larger batches run in chunks of this size.
int gemv_mfma_max_rows();
// The batched path reads Q4_0 / Q8_0 matrices from a tile-order copy (w->tiled, tiled_bytes(w)
// bytes).  ensure_tiled makes it when missing (allocates; refused while `s` is capturing a graph).
// refresh_tiled rewrites an existing copy from the handle's current bytes, in place and
// stream-ordered on `s` (no allocation, so graphs that read the copy stay valid); no-op without one.
size_t tiled_bytes(const ef_hip_weight_s* w);
int ensure_tiled(const ef_hip_weight_s* w, hipStream_t s);
int refresh_tiled(const ef_hip_weight_s* w, hipStream_t s);
int launch_gemv_mfma(const GemvJob* jobs, int n_jobs, int epi, const float* norm_w, float eps, int batch, size_t ldx,
                     size_t ldy, void* ws, size_t ws_bytes, hipStream_t stream, bool* taken);

// Batched products over K = 2048 that read the packed rows in place, in one launch with no
// workspace (gemv_batch.hip).  Sets *taken when it enqueued the launch; otherwise the caller takes
// another path.
int launch_gemv_batch(const GemvJob* jobs, int n_jobs, int epi, const float* norm_w, float eps, int batch,
                      size_t ldx, size_t ldy, hipStream_t stream, bool* taken);

// Block-scaled A tables of the matrix-core GEMV, staged by the kernel that produces its input
// (or by launch_stage_tables): t4 / t8 in the Q4_0 / Q8_0 column orders
// ([sequence tile][block][hi, lo][64 lanes][16 B], stage_table_bytes each), a power-of-two scale
// per (block, sequence) at bscale[block * bpad + sequence] (bpad >= stage_bpad(batch)), and for a
// product with an input RMSNorm n_ssp partial sums of squares of the un-normed input per sequence
// at ssp[p * bpad + sequence] (the tables then hold norm_w * x; 1 / rms scales the results).
struct MfmaStage {
  const uint8_t* t4 = nullptr;
  const uint8_t* t8 = nullptr;
  const float* bscale = nullptr;
  int bpad = 0;
  const double* ssp = nullptr;
  int n_ssp = 0;
  float eps = 0.0f;
};
constexpr int kStageMaxK = 8192;  // longest K launch_stage_tables prepares
size_t stage_table_bytes(int K, int batch);
int stage_bpad(int batch);
// The tables from x [batch][ldx] (one partial sum per sequence; norm_w may be null).
int launch_stage_tables(const float* x, size_t ldx, int K, int batch, const float* norm_w, const MfmaStage& st,
                        hipStream_t stream);
// The batched product over staged tables (one launch of <= 1024 sequences; ws as for launch_gemv,
// gemv_mfma_workspace_bytes of the same jobs).  With em on (one job whose rows are the next
// product's K), its outputs are also staged as that product's tables (afrag.h).
// Workspace of launch_gemv_mfma_staged (0: no matrix-core plan; emit: the launch stages its outputs).
size_t gemv_mfma_staged_workspace_bytes(const GemvJob* jobs, int n_jobs, int epi, int batch, bool emit);
int launch_gemv_mfma_staged(const GemvJob* jobs, int n_jobs, int epi, const MfmaStage& st, int batch, size_t ldy,
                            void* ws, size_t ws_bytes, hipStream_t stream, const AEmit* em = nullptr);

// F32 / F16 / BF16 weights (gemv_dense.hip): same jobs, epilogues and fused RMSNorm, any cols up to
// kMaxDenseCols; all jobs of one launch share the type.  launch_gemv routes these types here.
constexpr size_t kMaxDenseCols = 16320;
bool is_dense_qtype(int qtype);
int launch_gemv_dense(const GemvJob* jobs, int n_jobs, int epi, const float* norm_w, float eps, int batch,
                      size_t ldx, size_t ldy, hipStream_t stream);

// Any storage type.  Jobs of one launch share cols (and x); a launch that mixes packed and
// unquantized matrices is split into one launch per kind.
int launch_gemv(const GemvJob* jobs, int n_jobs, int epi, const float* norm_w, float eps, int batch, size_t ldx,
                size_t ldy, hipStream_t stream, void* ws = nullptr, size_t ws_bytes = 0);

}  // namespace efh
